// Full-order sampling path for bf16 logits: rows whose top-k is disabled or
// larger than the selection path's kMaxTopK (src/generation.cpp:80, k = V when
// top_k == 0). The reference sorts the whole row, takes an fp32 exp of every
// logit, sums them in double, and runs its top-p cumulative and the draw's
// subtract walk as fp32 left-to-right sums over the sorted probabilities
// (src/generation.cpp:79-126). With k = V the nucleus can hold most of the
// row, and those fp32 sums drift far from the exact ones, so the result
// depends on every rounding of the sequence.
//
// A bf16 row has at most 65536 distinct raw values, and every token of one
// value has the same final value and probability. Two kernels exploit that:
//
// fo_hist_kernel — one 1024-thread workgroup per row:
//   1. marks the row's unique history ids in a per-row device bitmap and
//      collects them (penalised tokens: their final value no longer follows
//      their raw bin), sorts them by (final value desc, index asc) in LDS;
//   2. streams the row once with 16-byte loads and counts every other token
//      in an LDS histogram over the 16-bit bf16 order key (two 16-bit
//      counters per word; a sweep every 32768 tokens moves counts that
//      reach 32768 to a spill list, so no counter wraps);
//   3. compacts the histogram into "items" (final value, count) in
//      descending order, merged with the penalised tokens, plus one NaN item
//      last.
// fo_decide_kernel — one 1024-thread workgroup per row:
//   4. evaluates expf per item, the double denominator (a parallel exact sum
//      when every partial sum is representable, else a closed-form replay),
//      the probabilities and the min-p cut;
//   5. replays the fp32 top-p cumulative and the subtract walk in closed form
//      (chain_math.h), one wave, 64 items at a time;
//   6. finds the chosen position's token: the n-th lowest index among the
//      tokens of the selected value, scanning the row from the nearer end.
//
// Selection is identical to sorting by (final value desc, index asc) — the
// lowest-index tie rule used everywhere in this library.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <type_traits>

#include "chain_block.h"
#include "chain_math.h"
#include "chain_wave.h"
#include "ge_math.h"
#include "sampler_internal.h"

#pragma clang fp contract(off)

namespace ge {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kSubChunk = 32768;          // tokens between overflow sweeps
constexpr uint32_t kWords = 32768;        // histogram words (two bins each)
constexpr uint32_t kNanLowMax = 0x007Eu;  // bins <= this are NaN patterns
constexpr uint32_t kNanHighMin = 0xFF81u; // bins >= this are NaN patterns
constexpr uint32_t kLowBin = 0x007Fu;     // -inf
constexpr uint32_t kHighBin = 0xFF80u;    // +inf
constexpr int kSpillCap = 512;
constexpr uint64_t kSat = static_cast<uint64_t>(1) << 62;

enum : uint32_t {
    kMetaItems = 0, kMetaExtras = 1, kMetaNan = 2, kMetaStatus = 3,
    // sorted rows only: the top k's exps, from the sort kernel (their sum
    // as two words of a double, the lowest set bit, any NaN)
    kMetaSumLo = 4, kMetaSumHi = 5, kMetaMinLsb = 6, kMetaAnyNan = 7
};
// kStatusFallback: items of a flagged bf16 row, made by the fallback sort;
// kStatusSkip: a row the fallback pass leaves as the first pass wrote it.
enum : uint32_t { kStatusOk = 0, kStatusTooManyPenalised = 1, kStatusFallback = 2, kStatusSkip = 3 };

// ---- bf16 order-key bins ---------------------------------------------------

__device__ __forceinline__ uint32_t bin_of(uint32_t bits16) {
    return (bits16 & 0x8000u) ? (~bits16 & 0xFFFFu) : (bits16 | 0x8000u);
}
__device__ __forceinline__ uint32_t bits_of_bin(uint32_t bin) {
    return (bin & 0x8000u) ? (bin & 0x7FFFu) : (~bin & 0xFFFFu);
}
__device__ __forceinline__ bool bin_is_nan(uint32_t bin) { return bin <= kNanLowMax || bin >= kNanHighMin; }
__device__ __forceinline__ float bin_value(uint32_t bin, float cap) {
    return softcap(bf16_to_f32(static_cast<uint16_t>(bits_of_bin(bin))), cap);
}
// Order key of a bin's final value. Monotone non-decreasing over
// [kLowBin, kHighBin]: widening is monotone and glibc tanhf is monotone.
__device__ __forceinline__ uint32_t bin_key(uint32_t bin, float cap) { return order_key(bin_value(bin, cap)); }

// ---- small helpers ---------------------------------------------------------

__device__ __forceinline__ float load_value(const float* rowp, int i) { return rowp[i]; }
__device__ __forceinline__ float load_value(const uint16_t* rowp, int i) { return bf16_to_f32(rowp[i]); }

__device__ __forceinline__ ge_sample_params params_of(const DevArgs& a, int row) {
    return a.row_params ? a.row_params[row] : a.params;
}

// generation.cpp:66, :80 — rows this path serves: sampling (T > 0 or NaN) with k > kMaxTopK.
__device__ __forceinline__ bool full_order_row(const ge_sample_params& p, int V, uint32_t& k) {
    if (p.temperature <= 0.0f) return false;
    k = p.top_k ? min(p.top_k, static_cast<uint32_t>(V)) : static_cast<uint32_t>(V);
    return k > static_cast<uint32_t>(kMaxTopK);
}

__device__ __forceinline__ void history_of(const DevArgs& a, int row, const int32_t*& h, int& n) {
    h = nullptr;
    n = 0;
    if (a.ring) {
        h = a.ring + static_cast<int64_t>(row) * a.ring_capacity;
        n = min(max(a.ring_len[row], 0), a.ring_capacity);
    } else if (a.history && a.history_offsets) {
        const int s = a.history_offsets[row];
        h = a.history + s;
        n = max(a.history_offsets[row + 1] - s, 0);
    }
}

__device__ __forceinline__ uint32_t rl32(uint32_t v, int lane) {
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), lane));
}
__device__ __forceinline__ uint64_t rl64(uint64_t v, int lane) {
    const uint32_t lo = rl32(static_cast<uint32_t>(v), lane);
    const uint32_t hi = rl32(static_cast<uint32_t>(v >> 32), lane);
    return (static_cast<uint64_t>(hi) << 32) | lo;
}
// v with lane kLane replaced by the wave-uniform x (v_writelane_b32; gfx950
// reads one SGPR per VALU instruction, so the lane is an immediate).
template <int kLane>
__device__ __forceinline__ uint64_t writelane64(uint64_t v, uint64_t x) {
    uint32_t lo = static_cast<uint32_t>(v), hi = static_cast<uint32_t>(v >> 32);
    asm("v_writelane_b32 %0, %1, %2" : "+v"(lo) : "s"(static_cast<uint32_t>(x)), "n"(kLane));
    asm("v_writelane_b32 %0, %1, %2" : "+v"(hi) : "s"(static_cast<uint32_t>(x >> 32)), "n"(kLane));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}
// f(std::integral_constant<int, J>) for J = J0 .. N - 1.
template <int J0, int N, typename F>
__device__ __forceinline__ void unroll_for(F&& f) {
    if constexpr (J0 < N) {
        f(std::integral_constant<int, J0>{});
        unroll_for<J0 + 1, N>(f);
    }
}
// Set bits of m below this lane.
__device__ __forceinline__ uint32_t lanes_below_u64(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
}
__device__ __forceinline__ double rld(double v, int lane) {
    return __builtin_bit_cast(double, rl64(__builtin_bit_cast(uint64_t, v), lane));
}

// Wave-wide inclusive scans with DPP (no LDS round trips): row_shr 1, 2, 4,
// 8 scan each row of 16 lanes (lanes shifted in from outside the row read
// 0), then row_bcast 15 / 31 carry row totals into rows 1, 3 and 2, 3.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(x), kCtrl, kRowMask, 0xf, true));
}
template <int kCtrl, int kRowMask>
__device__ __forceinline__ double dpp_f64(double x) {
    const uint64_t b = __builtin_bit_cast(uint64_t, x);
    const uint32_t lo = dpp_u32<kCtrl, kRowMask>(static_cast<uint32_t>(b));
    const uint32_t hi = dpp_u32<kCtrl, kRowMask>(static_cast<uint32_t>(b >> 32));
    return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}
constexpr int kRowShr1 = 0x111, kRowShr2 = 0x112, kRowShr4 = 0x114, kRowShr8 = 0x118;
constexpr int kRowBcast15 = 0x142, kRowBcast31 = 0x143;

__device__ __forceinline__ uint32_t wave_incl_u32(uint32_t v) {
    v += dpp_u32<kRowShr1, 0xf>(v);
    v += dpp_u32<kRowShr2, 0xf>(v);
    v += dpp_u32<kRowShr4, 0xf>(v);
    v += dpp_u32<kRowShr8, 0xf>(v);
    v += dpp_u32<kRowBcast15, 0xa>(v);
    v += dpp_u32<kRowBcast31, 0xc>(v);
    return v;
}

// Exact while every partial sum stays below 2^53.
__device__ __forceinline__ double wave_incl_f64(double v) {
    v += dpp_f64<kRowShr1, 0xf>(v);
    v += dpp_f64<kRowShr2, 0xf>(v);
    v += dpp_f64<kRowShr4, 0xf>(v);
    v += dpp_f64<kRowShr8, 0xf>(v);
    v += dpp_f64<kRowBcast15, 0xa>(v);
    v += dpp_f64<kRowBcast31, 0xc>(v);
    return v;
}

__device__ __forceinline__ uint64_t sat_add(uint64_t x, uint64_t y) {
    const uint64_t s = x + y;  // both <= kSat: no wrap
    return s > kSat ? kSat : s;
}

__device__ __forceinline__ uint64_t wave_incl_u64_sat(uint64_t v) {
    const int lane = __lane_id();
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint64_t t = __shfl_up(v, d, 64);
        if (lane >= d) v = sat_add(v, t);
    }
    return v;
}

__device__ __forceinline__ uint64_t sat_mul(uint64_t n, uint64_t d) {
    const uint64_t lo = n * d;
    return (__umul64hi(n, d) != 0 || lo > kSat) ? kSat : lo;
}

// Elements of an item (first element `first`, `n` elements) inside the top k.
// The saturating subtract is spelled as the builtin: clang has folded the
// form `first >= k ? 0 : min(n, k - first)` into an unguarded `k - first`
// marked no-wrap, so items past k were counted.
__device__ __forceinline__ uint32_t top_k_count(uint32_t first, uint32_t n, uint32_t k) {
    return min(n, __builtin_elementwise_sub_sat(k, first));
}

__device__ __forceinline__ int lsb_exp(float x) {  // exponent of the lowest set bit, x > 0 finite
    const uint32_t b = f2u(x);
    const uint32_t ex = b >> 23;
    const uint32_t man = b & 0x7fffffu;
    if (ex == 0) return -149 + __builtin_ctz(man);
    return static_cast<int>(ex) - 150 + __builtin_ctz(man | 0x800000u);
}

__device__ __forceinline__ int exp_of(double d) {  // floor(log2 d), d > 0 normal
    return static_cast<int>((__builtin_bit_cast(uint64_t, d) >> 52) & 0x7ff) - 1023;
}

// ---- kernel 1: histogram and item list --------------------------------------

struct HistShared {
    union {
        uint64_t sortkeys[kFoExtrasCap];  // penalised tokens: ids, then composite keys
        uint32_t hist[kWords];            // two 16-bit counters per word
    };
    uint16_t thr_bin[kFoExtrasCap];       // lowest bin whose final value is >= the token's
    uint32_t off[kThreads];               // items before each group of 64 bins
    uint64_t mask[kThreads];              // each group's non-empty, non-NaN bins
    uint32_t spill[kSpillCap];            // bins that moved 32768 counts out of LDS
    uint32_t scan[kWaves];
    uint32_t counters[4];                 // [0] penalised tokens, [1] spills, [2] NaN tokens
};

// After streaming, a bin's count is its LDS field plus 32768 per spill-list entry.
__device__ __forceinline__ uint32_t bin_spilled(const HistShared& sh, uint32_t bin, uint32_t nspill) {
    uint32_t c = 0;
    for (uint32_t i = 0; i < nspill; ++i) c += sh.spill[i] == bin ? 32768u : 0u;
    return c;
}

// Counts two bf16 tokens (one 32-bit word) without branches: a token with
// sign s and bits x has bin x | 0x8000 (s = 0: high field of word x & 0x7FFF)
// or ~x & 0xFFFF (s = 1: low field of word (x ^ 0x7FFF) & 0x7FFF). skip bit 0 /
// bit 1 drop the low / high token.
__device__ __forceinline__ void count_pair(HistShared& sh, uint32_t x, uint32_t skip) {
    const uint32_t sg = (x >> 15) & 0x00010001u;
    const uint32_t y = x ^ (sg * 0x7FFFu);
    const uint32_t inc_lo = (skip & 1u) ? 0u : (0x10000u >> ((sg & 1u) << 4));
    const uint32_t inc_hi = (skip & 2u) ? 0u : (0x10000u >> ((sg >> 16) << 4));
    atomicAdd(&sh.hist[y & 0x7FFFu], inc_lo);
    atomicAdd(&sh.hist[(y >> 16) & 0x7FFFu], inc_hi);
}

// Moves every field that reached 32768 to the spill list. At most kSubChunk
// counts arrive between sweeps, so a field below 32768 after a sweep cannot
// pass 65535 before the next one. Reads four words at a time and rejects
// them together in the common case that no field has its top bit set.
__device__ __forceinline__ void sweep(HistShared& sh, int tid) {
    __syncthreads();
    uint4* h4 = reinterpret_cast<uint4*>(sh.hist);
    for (uint32_t q = tid; q < kWords / 4; q += kThreads) {
        const uint4 x4 = h4[q];
        if (((x4.x | x4.y | x4.z | x4.w) & 0x80008000u) == 0u) continue;
        const uint32_t xs[4] = {x4.x, x4.y, x4.z, x4.w};
        for (int i = 0; i < 4; ++i) {
            const uint32_t w = 4 * q + i;
            const uint32_t x = xs[i];
            uint32_t sub = 0;
            if ((x & 0xFFFFu) >= 0x8000u) {
                sub += 0x8000u;
                const uint32_t sp = atomicAdd(&sh.counters[1], 1u);
                if (sp < kSpillCap) sh.spill[sp] = w;
            }
            if ((x >> 16) >= 0x8000u) {
                sub += 0x80000000u;
                const uint32_t sp = atomicAdd(&sh.counters[1], 1u);
                if (sp < kSpillCap) sh.spill[sp] = w + kWords;
            }
            if (sub) sh.hist[w] = x - sub;
        }
    }
    __syncthreads();
}

// Streams one row into the histogram. PEN: skip the tokens marked in the
// row's history bitmap. The loop is software-pipelined: the next sub-chunk's
// 16-byte loads are in flight while this one is counted and swept (the two
// variants keep the bitmap loads out of the unpenalised loop, so its wait
// counts only cover the data being counted).
template <bool PEN>
__device__ __forceinline__ void stream_row(HistShared& sh, const uint16_t* rowp, int V, bool vec,
                                           const uint32_t* bitmap, int tid) {
    constexpr int kVec = kSubChunk / (kThreads * 8);  // uint4 of 8 tokens per thread per sub-chunk
    const int vec_end = vec ? (V / kSubChunk) * kSubChunk : 0;
    if (vec_end > 0) {
        uint4 cur[kVec];
        uint32_t cbm[kVec];
#pragma unroll
        for (int j = 0; j < kVec; ++j) {
            const int pos = (j * kThreads + tid) * 8;
            cur[j] = *reinterpret_cast<const uint4*>(rowp + pos);
            cbm[j] = PEN ? (bitmap[pos >> 5] >> (pos & 31)) : 0u;
        }
        auto count_cur = [&]() {
#pragma unroll
            for (int j = 0; j < kVec; ++j) {
                count_pair(sh, cur[j].x, cbm[j] & 3u);
                count_pair(sh, cur[j].y, (cbm[j] >> 2) & 3u);
                count_pair(sh, cur[j].z, (cbm[j] >> 4) & 3u);
                count_pair(sh, cur[j].w, (cbm[j] >> 6) & 3u);
            }
        };
        // Two sub-chunks ahead: cur is counted while nxt and nxt2 load.
        uint4 nxt[kVec];
        uint32_t nbm[kVec];
        auto load_into = [&](uint4* q, uint32_t* bm, int base) {
#pragma unroll
            for (int j = 0; j < kVec; ++j) {
                const int pos = base + (j * kThreads + tid) * 8;
                q[j] = *reinterpret_cast<const uint4*>(rowp + pos);
                bm[j] = PEN ? (bitmap[pos >> 5] >> (pos & 31)) : 0u;
            }
        };
        if (kSubChunk < vec_end) load_into(nxt, nbm, kSubChunk);
        int base = 0;
        for (; base + 2 * kSubChunk < vec_end; base += kSubChunk) {
            uint4 nxt2[kVec];
            uint32_t nbm2[kVec];
            load_into(nxt2, nbm2, base + 2 * kSubChunk);
            count_cur();
            sweep(sh, tid);
#pragma unroll
            for (int j = 0; j < kVec; ++j) {
                cur[j] = nxt[j];
                cbm[j] = nbm[j];
                nxt[j] = nxt2[j];
                nbm[j] = nbm2[j];
            }
        }
        if (base + kSubChunk < vec_end) {  // second to last
            count_cur();
            sweep(sh, tid);
#pragma unroll
            for (int j = 0; j < kVec; ++j) {
                cur[j] = nxt[j];
                cbm[j] = nbm[j];
            }
        }
        count_cur();
        sweep(sh, tid);
    }
    for (int base = vec_end; base < V; base += kSubChunk) {
        for (int j = 0; j < kSubChunk / kThreads; ++j) {
            const int idx = base + j * kThreads + tid;
            if (idx < V) {
                const bool skip = PEN && ((bitmap[idx >> 5] >> (idx & 31)) & 1u);
                count_pair(sh, rowp[idx], skip ? 3u : 2u);  // the pair's high token is empty
            }
        }
        sweep(sh, tid);
    }
}

__global__ __launch_bounds__(kThreads) void fo_hist_kernel(DevArgs a) {
    __shared__ HistShared sh;
    const int tid = threadIdx.x;
    const int row = blockIdx.x;
    const int V = a.vocab;
    const ge_sample_params p = params_of(a, row);
    uint32_t k;
    if (!full_order_row(p, V, k) || row_done(a, row)) return;  // done rows: fo_decide_kernel reports them

    const uint16_t* rowp = static_cast<const uint16_t*>(a.logits) + static_cast<int64_t>(row) * a.row_stride;
    const int32_t* hist;
    int H;
    history_of(a, row, hist, H);
    const float r = p.repetition_penalty;
    const float cap = p.softcap;
    const bool pen = H > 0 && !(r == 1.0f);
    uint32_t* bitmap = a.fo_bitmap + static_cast<int64_t>(row) * a.fo_bitmap_words;
    uint64_t* extras = a.fo_extras + static_cast<int64_t>(row) * a.fo_extras_cap;
    uint64_t* items = a.fo_items + static_cast<int64_t>(row) * a.fo_items_stride;
    uint32_t* meta = a.fo_meta + static_cast<int64_t>(row) * kMetaWords;
    const uint32_t ecap = static_cast<uint32_t>(a.fo_extras_cap);

    if (tid < 4) sh.counters[tid] = 0;
    __syncthreads();

    // 1. Unique in-range history ids. The bitmap bits stay set until the
    //    decide kernel has used them and clears them.
    if (pen) {
        for (int i = tid; i < H; i += kThreads) {
            const int32_t id = hist[i];
            if (id < 0 || id >= V) continue;
            const uint32_t bit = 1u << (id & 31);
            const uint32_t old = atomicOr(&bitmap[id >> 5], bit);
            if (!(old & bit)) {
                const uint32_t e = atomicAdd(&sh.counters[0], 1u);
                if (e < ecap) sh.sortkeys[e] = static_cast<uint64_t>(id);
            }
        }
    }
    __syncthreads();
    const uint32_t e_all = sh.counters[0];
    if (e_all > ecap) {
        if (tid == 0) {
            meta[kMetaItems] = 0;
            meta[kMetaExtras] = 0;
            meta[kMetaNan] = 0;
            meta[kMetaStatus] = kStatusTooManyPenalised;
        }
        return;
    }
    const uint32_t E = e_all;

    // Final values of the penalised tokens, sorted (value desc, index asc),
    // and for each the lowest bin whose final value is >= its own.
    if (E > 0) {
        uint32_t n2 = 1;
        while (n2 < E) n2 <<= 1;
        for (uint32_t e = tid; e < n2; e += kThreads) {
            if (e < E) {
                const uint32_t id = static_cast<uint32_t>(sh.sortkeys[e]);
                const float v = penalize(softcap(bf16_to_f32(rowp[id]), cap), r);
                sh.sortkeys[e] = composite(order_key(v), id);
            } else {
                sh.sortkeys[e] = 0;  // sorts last
            }
        }
        __syncthreads();
        for (uint32_t size = 2; size <= n2; size <<= 1) {
            for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
                for (uint32_t i = tid; i < n2; i += kThreads) {
                    const uint32_t j = i ^ stride;
                    if (j > i) {
                        const uint64_t x = sh.sortkeys[i];
                        const uint64_t y = sh.sortkeys[j];
                        const bool desc = (i & size) == 0;
                        if (desc ? (x < y) : (x > y)) {
                            sh.sortkeys[i] = y;
                            sh.sortkeys[j] = x;
                        }
                    }
                }
                __syncthreads();
            }
        }
        for (uint32_t e = tid; e < E; e += kThreads) {
            const uint64_t c = sh.sortkeys[e];
            extras[e] = c;
            const uint32_t key = composite_key(c);
            // lowest bin b in [kLowBin, kHighBin] with bin_key(b) >= key
            uint32_t lo = kLowBin, hi = kHighBin + 1;
            while (lo < hi) {
                const uint32_t mid = (lo + hi) >> 1;
                if (bin_key(mid, cap) >= key) hi = mid;
                else lo = mid + 1;
            }
            sh.thr_bin[e] = static_cast<uint16_t>(lo);  // kHighBin + 1 when none
        }
    }
    __syncthreads();

    // 2. Histogram of the non-penalised tokens.
    for (uint32_t w = tid; w < kWords; w += kThreads) sh.hist[w] = 0u;
    __syncthreads();

    if (pen) stream_row<true>(sh, rowp, V, a.vec_ok != 0, bitmap, tid);
    else stream_row<false>(sh, rowp, V, a.vec_ok != 0, bitmap, tid);
    const uint32_t nspill = min(sh.counters[1], static_cast<uint32_t>(kSpillCap));

    // 3. Items in descending order. After the last sweep every field is below
    //    0x8000, so bit 15 can mark the bins of the spill list: a spilled bin
    //    whose field is 0 then still reads as non-empty.
    for (uint32_t i = tid; i < nspill; i += kThreads) {
        const uint32_t e = sh.spill[i];
        atomicOr(&sh.hist[e & (kWords - 1)], 0x8000u << ((e / kWords) * 16u));
    }
    __syncthreads();
    //    Wave w owns histogram words kWords - 1 - 2048 w - 64 j - l for
    //    j = 0..31 (group) and l = 0..63 (lane); word x holds the "high" bin
    //    x + kWords (upper field) and the "low" bin x (lower field). Bins in
    //    descending order are the high bins by descending word, then the low
    //    bins by descending word, i.e. (wave, group, lane) order in each half.
    //    Lane j keeps group j's two ballots; sh.mask / sh.off hold them with
    //    the items before each group, high groups at [0, 512), low at [512, 1024).
    const int lane = __lane_id();
    const int wave = tid >> 6;
    const uint32_t wtop = (kWords - 1u) - 2048u * static_cast<uint32_t>(wave);
    uint32_t words[32];  // this lane's histogram words
#pragma unroll
    for (int j = 0; j < 32; ++j) words[j] = sh.hist[wtop - 64u * j - lane];
    auto field_count = [&](uint32_t f, uint32_t bin) {
        return (f & 0x7FFFu) + ((f & 0x8000u) ? bin_spilled(sh, bin, nspill) : 0u);
    };
    uint64_t mhi = 0, mlo = 0;
    uint32_t nan_local = 0;
    unroll_for<0, 32>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        const uint32_t x = words[j];
        bool nh = (x >> 16) != 0u;
        bool nl = (x & 0xFFFFu) != 0u;
        if ((wave == 0 && j < 2) || (wave == kWaves - 1 && j >= 30)) {  // the groups holding NaN bins
            const uint32_t w = wtop - 64u * j - lane;
            if (nh && bin_is_nan(w + kWords)) {
                nan_local += field_count(x >> 16, w + kWords);
                nh = false;
            }
            if (nl && bin_is_nan(w)) {
                nan_local += field_count(x & 0xFFFFu, w);
                nl = false;
            }
        }
        const uint64_t bh = __ballot(nh);
        const uint64_t bl = __ballot(nl);
        mhi = writelane64<j>(mhi, bh);
        mlo = writelane64<j>(mlo, bl);
    });
    const uint32_t ph = static_cast<uint32_t>(__popcll(mhi));  // lanes past 31: 0
    const uint32_t pl = static_cast<uint32_t>(__popcll(mlo));
    const uint32_t ih = wave_incl_u32(ph);
    const uint32_t il = wave_incl_u32(pl);
    if (lane == 63) sh.scan[wave] = (ih << 16) | il;  // each at most 2048
    if (nan_local) atomicAdd(&sh.counters[2], nan_local);
    __syncthreads();  // also: every histogram word is read
    uint32_t tot_hi = 0, tot_lo = 0, before_hi = 0, before_lo = 0;
    for (int w = 0; w < kWaves; ++w) {
        const uint32_t x = sh.scan[w];
        if (w < wave) {
            before_hi += x >> 16;
            before_lo += x & 0xFFFFu;
        }
        tot_hi += x >> 16;
        tot_lo += x & 0xFFFFu;
    }
    const uint32_t nbins_total = tot_hi + tot_lo;
    const uint32_t ohi = before_hi + ih - ph;
    const uint32_t olo = tot_hi + before_lo + il - pl;
    if (lane < 32) {
        sh.mask[wave * 32 + lane] = mhi;
        sh.mask[512 + wave * 32 + lane] = mlo;
        sh.off[wave * 32 + lane] = ohi;
        sh.off[512 + wave * 32 + lane] = olo;
    }
    __syncthreads();

    // Bin items, spread over the waves by group (group g goes to wave g % 16,
    // so the few dense groups of a typical row land on different waves): a
    // lane with a non-empty bin writes its final value and count at its rank
    // among the bins plus the penalised tokens above it. Lane i of a wave
    // prefetches the wave's i-th group; four groups are taken per round so
    // that their softcap chains overlap.
    {
        const uint32_t gl = static_cast<uint32_t>(wave) + 16u * static_cast<uint32_t>(lane);
        const uint64_t gm = sh.mask[gl];
        const uint32_t go = sh.off[gl];
        uint64_t todo = __ballot(gm != 0ull);
        while (todo) {
            constexpr int kRound = 4;
            uint32_t bin[kRound], cnt[kRound], r[kRound];
            bool on[kRound];
#pragma unroll
            for (int u = 0; u < kRound; ++u) {
                on[u] = false;
                bin[u] = kLowBin;
                cnt[u] = 0;
                r[u] = 0;
                if (todo == 0ull) continue;  // wave-uniform
                const int i = __builtin_ctzll(todo);
                todo &= todo - 1ull;
                const uint64_t m = wave::readlane64(gm, i);
                on[u] = ((m >> lane) & 1u) != 0u;
                const uint32_t g = static_cast<uint32_t>(wave) + 16u * static_cast<uint32_t>(i);
                const bool high = g < 512u;
                const uint32_t word = (kWords - 1u) - 2048u * ((g & 511u) >> 5) - 64u * (g & 31u) - lane;
                bin[u] = high ? word + kWords : word;
                if (on[u]) {
                    const uint32_t x = sh.hist[word];
                    cnt[u] = field_count(high ? (x >> 16) : (x & 0xFFFFu), bin[u]);
                }
                r[u] = rl32(go, i) + lanes_below_u64(m);
            }
            float v[kRound];
#pragma unroll
            for (int u = 0; u < kRound; ++u) v[u] = bin_value(bin[u], cap);
#pragma unroll
            for (int u = 0; u < kRound; ++u) {
                if (!on[u]) continue;
                uint32_t lo = 0, hi = E;  // penalised tokens with thr_bin > bin (thr_bin is non-increasing)
                while (lo < hi) {
                    const uint32_t mid = (lo + hi) >> 1;
                    if (sh.thr_bin[mid] > bin[u]) lo = mid + 1;
                    else hi = mid;
                }
                items[r[u] + lo] = (static_cast<uint64_t>(f2u(v[u])) << 32) | cnt[u];
            }
        }
    }
    // Penalised items: position = own rank + bins with a final value >= its own.
    for (uint32_t e = tid; e < E; e += kThreads) {
        const uint32_t tb = sh.thr_bin[e];
        uint32_t nb = 0;
        if (tb <= kHighBin) {  // bins >= tb: in tb's half, the words >= tb's word
            const uint32_t d = (kWords - 1u) - (tb & (kWords - 1u));
            const uint32_t g = (tb >= kWords ? 0u : 512u) + (d >> 6);  // group holding tb
            const uint32_t l = d & 63u;                                // its lane
            const uint64_t upto = l == 63 ? ~0ull : ((2ull << l) - 1);
            nb = sh.off[g] + static_cast<uint32_t>(__popcll(sh.mask[g] & upto));
        }
        const uint32_t key = composite_key(extras[e]);
        items[e + nb] = (static_cast<uint64_t>(f2u(key_value(key))) << 32) | 1u;
    }
    const uint32_t nan_total = sh.counters[2];
    if (tid == 0) {
        uint32_t g = nbins_total + E;
        if (nan_total) items[g++] = (static_cast<uint64_t>(0x7fc00000u) << 32) | nan_total;
        meta[kMetaItems] = g;
        meta[kMetaExtras] = E;
        meta[kMetaNan] = nan_total;
        meta[kMetaStatus] = kStatusOk;
    }
}

// ---- kernel 1, f32 rows: every token's final key, sorted --------------------
//
// An f32 row can hold V distinct values, so its items come from a sort of
// the final keys of all its tokens (softcap, then the penalty on marked ids),
// complemented so that ascending order is the reference's descending one.
// One 1024-thread workgroup per row runs a stable LSD radix sort, 8 bits per
// pass, ping-ponging between two per-row buffers in global memory (the decide
// kernel's aux and pre arrays, unused until then). The four digit histograms
// are counted once, while the keys are made. Each pass takes the row in tiles
// of 16384 keys in order: every wave ranks its 512 consecutive keys per digit
// (ballots over the digit's bits give the ranks among the 64 lanes of a step;
// per-wave LDS counters carry them across steps), the tile's keys are then
// placed in LDS grouped by digit, and the block writes each digit's group to
// its place in the output, so consecutive threads store consecutive
// addresses. Runs of equal keys then become the items (value, count).

constexpr int kDigits = 256;
constexpr int kSortUnroll = 8;  // 64-token steps in flight per wave
constexpr int kTileSteps = 16;  // 64-key steps per wave per tile
constexpr int kTileKeys = kThreads * kTileSteps;

struct SortShared {
    uint32_t staged[kTileKeys];       // the tile's keys grouped by digit
    uint32_t wc[kWaves][kDigits];     // per wave: keys of each digit so far in the tile, then its offset
    uint32_t hist[4][kDigits];        // the row's four digit histograms
    uint32_t gbase[kDigits];          // next output position of each digit
    uint32_t toff[kDigits];           // first staged position of each digit in the tile
    uint32_t scan[kWaves];
    double dred[kWaves];              // per-wave sums, lowest set bits, NaN flags of the exps
    int ired[kWaves];
    uint32_t ured[kWaves];
};

// Buffer reads of the sort read from L2 (agent-scope loads skip the CU's L1),
// so a line the L1 kept from an earlier pass is never used after another wave
// of the workgroup rewrote it; the writers wait for their stores before each
// barrier.
__device__ __forceinline__ uint32_t ld_l2(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stores_done_barrier() {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
}

// Lanes among `act` whose 8-bit digit equals this lane's.
__device__ __forceinline__ uint64_t match_digit(uint32_t d, uint64_t act) {
    uint64_t m = act;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const bool bit = ((d >> b) & 1u) != 0u;
        const uint64_t bb = __ballot(bit);
        m &= bit ? bb : ~bb;
    }
    return m;
}

// Exclusive prefix over the 256 digits of v (one value per thread tid < 256;
// the 4 waves holding them combine through scan[]), with the total.
__device__ __forceinline__ uint32_t digit_excl_scan(uint32_t v, uint32_t* scan, int tid) {
    const int lane = tid & 63, wave = tid >> 6;
    const uint32_t incl = wave_incl_u32(v);
    if (tid < kDigits && lane == 63) scan[wave] = incl;
    __syncthreads();
    uint32_t before = 0;
    for (int w = 0; w < wave && w < kDigits / 64; ++w) before += scan[w];
    return before + incl - v;
}

template <typename T>
__global__ __launch_bounds__(kThreads) void fo_sort_kernel(DevArgs a) {
    __shared__ SortShared sh;
    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int wave = tid >> 6;
    const int row = blockIdx.x;
    const int V = a.vocab;
    const ge_sample_params p = params_of(a, row);
    uint32_t k;
    if (!full_order_row(p, V, k) || row_done(a, row)) return;  // done rows: fo_decide_kernel reports them
    if (a.fo_fallback) {
        // Only rows the first pass flagged (its status word, at the call
        // row); the decide kernel of this pass skips the others.
        const uint32_t st = a.fo_meta[static_cast<int64_t>(a.fo_row0 + row) * kMetaWords + kMetaStatus];
        __syncthreads();  // every thread has read it before thread 0 may rewrite it below
        if (st != kStatusTooManyPenalised) {
            if (tid == 0) a.fo_meta[static_cast<int64_t>(row) * kMetaWords + kMetaStatus] = kStatusSkip;
            return;
        }
    }

    const T* rowp = static_cast<const T*>(a.logits) + static_cast<int64_t>(row) * a.row_stride;
    const int32_t* hist;
    int H;
    history_of(a, row, hist, H);
    const float r = p.repetition_penalty;
    const float cap = p.softcap;
    const bool pen = H > 0 && !(r == 1.0f);
    uint32_t* bitmap = a.fo_bitmap + static_cast<int64_t>(row) * a.fo_bitmap_words;
    uint64_t* items = a.fo_items + static_cast<int64_t>(row) * a.fo_items_stride;
    uint32_t* meta = a.fo_meta + static_cast<int64_t>(row) * kMetaWords;
    uint32_t* buf0 = reinterpret_cast<uint32_t*>(a.fo_aux) + static_cast<int64_t>(row) * a.fo_items_stride;
    uint32_t* buf1 = a.fo_pre + static_cast<int64_t>(row) * a.fo_items_stride;

    // 1. Unique in-range history ids; the decide kernel clears the bits.
    if (pen) {
        for (int i = tid; i < H; i += kThreads) {
            const int32_t id = hist[i];
            if (id >= 0 && id < V) atomicOr(&bitmap[id >> 5], 1u << (id & 31));
        }
    }
    for (int i = tid; i < 4 * kDigits; i += kThreads) (&sh.hist[0][0])[i] = 0u;
    stores_done_barrier();

    const uint64_t below = (1ull << lane) - 1ull;

    // 2. Final keys (generation.cpp:431-437 softcap, then the penalty) and the
    //    four digit histograms.
    for (int base = 0; base < V; base += kThreads * kSortUnroll) {
        float x[kSortUnroll];
        uint32_t bw[kSortUnroll];
#pragma unroll
        for (int u = 0; u < kSortUnroll; ++u) {
            const int i = base + u * kThreads + tid;
            const int ic = min(i, V - 1);  // clamped: no conditional load (values past V unused)
            x[u] = load_value(rowp, ic);
            bw[u] = pen ? ld_l2(bitmap + (ic >> 5)) : 0u;
        }
#pragma unroll
        for (int u = 0; u < kSortUnroll; ++u) {
            const int i = base + u * kThreads + tid;
            if (i < V) {
                float f = softcap(x[u], cap);
                if ((bw[u] >> (i & 31)) & 1u) f = penalize(f, r);
                const uint32_t s = ~order_key(f);
                buf0[i] = s;
#pragma unroll
                for (int b = 0; b < 4; ++b) atomicAdd(&sh.hist[b][(s >> (8 * b)) & 255u], 1u);
            }
        }
    }

    // 3. Four stable passes, least significant digit first.
    uint32_t* src = buf0;
    uint32_t* dst = buf1;
    const int ntiles = (V + kTileKeys - 1) / kTileKeys;
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 8 * pass;
        stores_done_barrier();  // histograms complete, the previous pass's stores done
        // (every thread takes part in the scan's barrier; gbase is first read
        // in step d, after three more)
        const uint32_t g0 = digit_excl_scan(tid < kDigits ? sh.hist[pass][tid] : 0u, sh.scan, tid);
        if (tid < kDigits) sh.gbase[tid] = g0;
        uint32_t key[kTileSteps], nkey[kTileSteps];
        auto load_tile = [&](int t, uint32_t* kv) {
#pragma unroll
            for (int u = 0; u < kTileSteps; ++u) {
                const int i = t * kTileKeys + wave * (64 * kTileSteps) + u * 64 + lane;
                kv[u] = ld_l2(src + min(i, V - 1));  // clamped: keys past V unused
            }
        };
        load_tile(0, key);
        uint32_t tot_prev = 0;  // (thread d < 256) keys of digit d in the previous tile
        for (int t = 0; t < ntiles; ++t) {
            if (t + 1 < ntiles) load_tile(t + 1, nkey);
            // a. Ranks among this wave's keys of the same digit, in position order.
            //    (The previous tile's step d read staged, gbase and toff before
            //    the barrier below; its readers of wc finished before step d.)
            for (int d = lane; d < kDigits; d += 64) sh.wc[wave][d] = 0u;  // only this wave uses its row
            uint32_t lr[kTileSteps];
#pragma unroll
            for (int u = 0; u < kTileSteps; ++u) {
                const int i = t * kTileKeys + wave * (64 * kTileSteps) + u * 64 + lane;
                const bool act = i < V;
                const uint64_t am = __ballot(act);
                const uint32_t d = (key[u] >> shift) & 255u;
                const uint64_t mm = match_digit(d, am);
                lr[u] = 0u;
                if (act) {
                    // Lanes of one digit read the same counter, then all write
                    // the same advanced value (in program order, so the next
                    // step reads it).
                    const uint32_t c = sh.wc[wave][d];
                    lr[u] = c + static_cast<uint32_t>(__popcll(mm & below));
                    sh.wc[wave][d] = c + static_cast<uint32_t>(__popcll(mm));
                }
            }
            __syncthreads();
            // b. Per digit: each wave's offset among the tile's keys of that
            //    digit, and the digit's first position in the staged tile.
            uint32_t tot = 0;
            if (tid < kDigits) {
                sh.gbase[tid] += tot_prev;  // the previous tile's keys of this digit are placed
                for (int w = 0; w < kWaves; ++w) {
                    const uint32_t c = sh.wc[w][tid];
                    sh.wc[w][tid] = tot;
                    tot += c;
                }
            }
            const uint32_t to = digit_excl_scan(tid < kDigits ? tot : 0u, sh.scan, tid);
            if (tid < kDigits) sh.toff[tid] = to;
            __syncthreads();
            // c. The tile's keys grouped by digit, in position order inside a group.
#pragma unroll
            for (int u = 0; u < kTileSteps; ++u) {
                const int i = t * kTileKeys + wave * (64 * kTileSteps) + u * 64 + lane;
                if (i < V) {
                    const uint32_t d = (key[u] >> shift) & 255u;
                    sh.staged[sh.toff[d] + sh.wc[wave][d] + lr[u]] = key[u];
                }
            }
            __syncthreads();
            // d. Each digit's group to its place in the output.
            const int nt = min(kTileKeys, V - t * kTileKeys);
#pragma unroll
            for (int u = 0; u < kTileSteps; ++u) {
                const int q = u * kThreads + tid;
                if (q < nt) {
                    const uint32_t kv = sh.staged[q];
                    const uint32_t d = (kv >> shift) & 255u;
                    dst[sh.gbase[d] + static_cast<uint32_t>(q) - sh.toff[d]] = kv;
                }
            }
            tot_prev = tot;
#pragma unroll
            for (int u = 0; u < kTileSteps; ++u) key[u] = nkey[u];
        }
        uint32_t* tmp = src;
        src = dst;
        dst = tmp;
    }
    stores_done_barrier();

    // Wave w owns positions [w P, (w + 1) P), P a power of two, in the items.
    int lgP = 6;
    while ((static_cast<int64_t>(kWaves) << lgP) < V) ++lgP;
    const int wlo = min(wave << lgP, V);
    const int whi = min(wlo + (1 << lgP), V);

    // 4. Items: runs of equal keys in the sorted order (src); their starts
    //    go to the other buffer.
    const uint32_t* s = src;
    uint32_t* istart = dst;
    // (kSortUnroll steps of loads in flight per wave)
    auto load_pairs = [&](int base, uint32_t* cv, uint32_t* pv) {
#pragma unroll
        for (int u = 0; u < kSortUnroll; ++u) {
            const int i = base + 64 * u + lane;
            const int ic = min(i, whi - 1);  // clamped: no conditional load (unused when i >= whi)
            cv[u] = ld_l2(s + ic);
            pv[u] = ld_l2(s + max(ic - 1, 0));
        }
    };
    uint32_t nb = 0;
    for (int base = wlo; base < whi; base += 64 * kSortUnroll) {
        uint32_t cv[kSortUnroll], pv[kSortUnroll];
        load_pairs(base, cv, pv);
#pragma unroll
        for (int u = 0; u < kSortUnroll; ++u) {
            const int i = base + 64 * u + lane;
            nb += static_cast<uint32_t>(__popcll(__ballot(i < whi && (i == 0 || cv[u] != pv[u]))));
        }
    }
    if (lane == 0) sh.scan[wave] = nb;
    __syncthreads();
    uint32_t j = 0, G = 0;
    for (int w = 0; w < kWaves; ++w) {
        const uint32_t x = sh.scan[w];
        if (w < wave) j += x;
        G += x;
    }
    for (int base = wlo; base < whi; base += 64 * kSortUnroll) {
        uint32_t cv[kSortUnroll], pv[kSortUnroll];
        load_pairs(base, cv, pv);
#pragma unroll
        for (int u = 0; u < kSortUnroll; ++u) {
            const int i = base + 64 * u + lane;
            const bool bnd = i < whi && (i == 0 || cv[u] != pv[u]);
            const uint64_t m = __ballot(bnd);
            if (bnd) istart[j + static_cast<uint32_t>(__popcll(m & below))] = static_cast<uint32_t>(i);
            j += static_cast<uint32_t>(__popcll(m));
        }
    }
    if (tid == 0) istart[G] = static_cast<uint32_t>(V);
    stores_done_barrier();
    // 5. The items (value, count), and each item's exp in aux for the decide
    //    kernel (generation.cpp:94-97: p = exp((l - max) * (1/T)), max the
    //    first item's value) with the certificate of their double sum over the
    //    top k (the sum, the lowest set bit, any NaN). aux holds the sorted
    //    keys being read: rounds of 16384 items read their keys, wait at a
    //    barrier, then write; later rounds read only keys at or after their
    //    own items' positions, past every position written before.
    const uint32_t key0 = ~ld_l2(s);
    const float vmax = key0 == kKeyNaN ? u2f(0x7fc00000u) : key_value(key0);
    const bool last_nan = ~ld_l2(s + V - 1) == kKeyNaN;  // (read before aux is rewritten)
    const float inv_temp = 1.0f / p.temperature;
    float* aux = a.fo_aux + static_cast<int64_t>(row) * a.fo_items_stride;
    double S = 0.0;
    int minlsb = INT_MAX;
    bool nan = false;
    constexpr int kQ = 16;
    for (uint32_t q0 = tid; q0 - tid < G; q0 += kThreads * kQ) {  // uniform trip count
        uint32_t st[kQ], en[kQ];
#pragma unroll
        for (int u = 0; u < kQ; ++u) {  // indices clamped to the last item: no conditional load
            const uint32_t q = min(q0 + u * kThreads, G - 1u);
            st[u] = ld_l2(istart + q);
            en[u] = ld_l2(istart + q + 1);
        }
        uint32_t kv[kQ];
#pragma unroll
        for (int u = 0; u < kQ; ++u) kv[u] = ld_l2(s + st[u]);
        // Every thread's key loads of this round have returned before any
        // thread writes aux: an item's first key can sit at the position of
        // a later item of the same round (a barrier alone does not wait for
        // loads in flight).
        stores_done_barrier();
#pragma unroll
        for (int u = 0; u < kQ; ++u) {
            const uint32_t q = q0 + u * kThreads;
            if (q < G) {
                const uint32_t key = ~kv[u];
                const uint32_t val = key == kKeyNaN ? 0x7fc00000u : f2u(key_value(key));
                const uint32_t n = en[u] - st[u];
                items[q] = (static_cast<uint64_t>(val) << 32) | n;
                const float pe = expf_glibc((u2f(val) - vmax) * inv_temp);
                aux[q] = pe;
                const uint32_t nk = top_k_count(st[u], n, k);
                if (nk) {
                    if (pe != pe) nan = true;
                    else if (pe > 0.0f) {
                        minlsb = min(minlsb, lsb_exp(pe));
                        S += static_cast<double>(nk) * static_cast<double>(pe);
                    }
                }
            }
        }
    }
    S = wave::sum_f64(S);  // a certificate: exact whenever it certifies
    minlsb = wave::min_i32(minlsb);
    const uint32_t nanw = __ballot(nan) != 0ull ? 1u : 0u;
    if (lane == 0) {
        sh.dred[wave] = S;
        sh.ired[wave] = minlsb;
        sh.ured[wave] = nanw;
    }
    __syncthreads();
    if (tid == 0) {
        double Sp = 0.0;
        int ml = INT_MAX;
        uint32_t nn = 0;
        for (int w = 0; w < kWaves; ++w) {
            Sp += sh.dred[w];
            ml = min(ml, sh.ired[w]);
            nn |= sh.ured[w];
        }
        const uint64_t sb = __builtin_bit_cast(uint64_t, Sp);
        meta[kMetaSumLo] = static_cast<uint32_t>(sb);
        meta[kMetaSumHi] = static_cast<uint32_t>(sb >> 32);
        meta[kMetaMinLsb] = static_cast<uint32_t>(ml);
        meta[kMetaAnyNan] = nn;
        meta[kMetaItems] = G;
        meta[kMetaExtras] = 0;
        meta[kMetaNan] = last_nan ? static_cast<uint32_t>(V) - ld_l2(istart + G - 1) : 0u;
        meta[kMetaStatus] = a.fo_fallback ? kStatusFallback : kStatusOk;
    }
}

// ---- f32 rows over many workgroups: the same items, tile by tile -----------
//
// The sort above gives each row one workgroup; with few rows most of the GPU
// idles while its passes run. Here a row's keys are cut into tiles of
// kSTile keys, one 256-thread workgroup per (tile, row), and each step of the
// sort is a kernel of its own: the kernel boundaries order every exchange
// between workgroups, so no workgroup waits for another. The results are
// those of fo_sort_kernel<float>: the sorted keys' items (value, count) in
// fo_items, their first elements in fo_pre (and pre[G] = V), their exps in
// fo_aux and the row's meta words; fo_decide_kernel<float, true> follows.
// Per row the tile area (fo_tiles) holds the (digit, tile) counts, then their
// output positions, the tiles' item counts and their certificate partials.

constexpr int kSThreads = 256;
constexpr int kSWaves = kSThreads / 64;
constexpr int kSSteps = 16;                     // 64-key steps per wave per tile
constexpr int kSTile = kSThreads * kSSteps;     // 4096 keys
constexpr int kKThreads = 1024;                  // fs_keys_kernel's workgroup
constexpr int kKSteps = kSTile / kKThreads;
static_assert(kKThreads >= kDigits && kSTile % kKThreads == 0, "the keys kernel's layout");
constexpr int64_t kSplitMaxRows = 160;          // larger f32 slices: fo_sort_kernel
constexpr int kSplitFuseRows = 8;               // slices up to this: no scan kernel

static_assert(kSTile == 4096, "fo_split_tiles() and fo_tile_words() assume 4096-key tiles");

// The row's tile area: counts [T][kDigits], item counts [T], partials [T][4].
struct SplitRow {
    uint32_t* cnt;
    uint32_t* bc;
    uint32_t* part;
};
__device__ __forceinline__ SplitRow split_row(const DevArgs& a, int row, int T) {
    uint32_t* w = a.fo_tiles + static_cast<int64_t>(row) * fo_tile_words(T);
    return SplitRow{w, w + kDigits * T, w + (kDigits + 1) * T};
}

// Rows this path serves (the sort kernel's condition).
__device__ __forceinline__ bool split_row_active(const DevArgs& a, int row, uint32_t& k, ge_sample_params& p) {
    p = params_of(a, row);
    return full_order_row(p, a.vocab, k) && !row_done(a, row);
}

// Items before tile t: the sum of the tiles' item counts (one wave).
__device__ __forceinline__ uint32_t items_before(const uint32_t* bc, int t) {
    uint32_t s = 0;
    for (int i = __lane_id(); i < t; i += 64) s += bc[i];
    return wave::readlane(wave::incl_add(s), 63);
}

// 1. The penalty bitmap of the row's unique in-range history ids (cleared by
//    the decide kernel).
__global__ __launch_bounds__(kSThreads) void fs_bitmap_kernel(DevArgs a) {
    const int row = blockIdx.x;
    uint32_t k;
    ge_sample_params p;
    if (!split_row_active(a, row, k, p)) return;
    const int32_t* hist;
    int H;
    history_of(a, row, hist, H);
    if (!(H > 0 && !(p.repetition_penalty == 1.0f))) return;
    uint32_t* bitmap = a.fo_bitmap + static_cast<int64_t>(row) * a.fo_bitmap_words;
    for (int i = threadIdx.x; i < H; i += kSThreads) {
        const int32_t id = hist[i];
        if (id >= 0 && id < a.vocab) atomicOr(&bitmap[id >> 5], 1u << (id & 31));
    }
}

// 2. Final keys (generation.cpp:431-437 softcap, then the penalty) of tile t
//    into buf0, and the tile's count of each lowest digit. With `fused` (a
//    few rows), the tile also builds its own words of the penalty bitmap from
//    the history (fs_bitmap_kernel is then not launched).
// (1024 threads: 16 waves per CU hide the softcap's dependent latency, where
// one wave per SIMD did not)
__global__ __launch_bounds__(kKThreads) void fs_keys_kernel(DevArgs a, int fused) {
    __shared__ uint32_t h[kDigits];
    __shared__ uint32_t tbits[kSTile / 32];
    const int t = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    uint32_t k;
    ge_sample_params p;
    if (!split_row_active(a, row, k, p)) return;
    const int V = a.vocab, T = gridDim.x;
    const int32_t* hist;
    int H;
    history_of(a, row, hist, H);
    const bool pen = H > 0 && !(p.repetition_penalty == 1.0f);
    const float* rowp = static_cast<const float*>(a.logits) + static_cast<int64_t>(row) * a.row_stride;
    uint32_t* bitmap = a.fo_bitmap + static_cast<int64_t>(row) * a.fo_bitmap_words;
    uint32_t* buf0 = reinterpret_cast<uint32_t*>(a.fo_aux) + static_cast<int64_t>(row) * a.fo_items_stride;
    if (tid < kDigits) h[tid] = 0u;
    const int lo = t * kSTile;
    if (fused && pen) {
        // this tile's bitmap words (a tile is a whole number of words); the
        // row's bitmap is all zero between calls
        for (int w = tid; w < kSTile / 32; w += kKThreads) tbits[w] = 0u;
        __syncthreads();
        const int hi = min(lo + kSTile, V);
        for (int i = tid; i < H; i += kKThreads) {
            const int32_t id = hist[i];
            if (id >= lo && id < hi) atomicOr(&tbits[(id - lo) >> 5], 1u << (id & 31));
        }
        __syncthreads();
        for (int w = tid; w < (hi - lo + 31) / 32; w += kKThreads) bitmap[(lo >> 5) + w] = tbits[w];
    }
    __syncthreads();
    float x[kKSteps];
    uint32_t bw[kKSteps];
#pragma unroll
    for (int u = 0; u < kKSteps; ++u) {
        const int i = t * kSTile + u * kKThreads + tid;
        const int ic = min(i, V - 1);  // clamped: no conditional load (values past V unused)
        x[u] = rowp[ic];
        bw[u] = pen ? (fused ? tbits[(ic - lo) >> 5] : bitmap[ic >> 5]) : 0u;
    }
#pragma unroll
    for (int u = 0; u < kKSteps; ++u) {
        const int i = t * kSTile + u * kKThreads + tid;
        if (i < V) {
            float f = softcap(x[u], p.softcap);
            if ((bw[u] >> (i & 31)) & 1u) f = penalize(f, p.repetition_penalty);
            const uint32_t s = ~order_key(f);
            buf0[i] = s;
            atomicAdd(&h[s & 255u], 1u);
        }
    }
    __syncthreads();
    if (tid < kDigits) split_row(a, row, T).cnt[t * kDigits + tid] = h[tid];
}

// 3a. The tile's count of each digit of pass `shift` (passes after the first).
__global__ __launch_bounds__(kKThreads) void fs_count_kernel(DevArgs a, int shift, int src_is_buf1) {  // (1024 threads)
    __shared__ uint32_t h[kDigits];
    const int t = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    uint32_t k;
    ge_sample_params p;
    if (!split_row_active(a, row, k, p)) return;
    const int V = a.vocab, T = gridDim.x;
    const uint32_t* src = src_is_buf1 ? a.fo_pre + static_cast<int64_t>(row) * a.fo_items_stride
                                      : reinterpret_cast<const uint32_t*>(a.fo_aux) + static_cast<int64_t>(row) * a.fo_items_stride;
    if (tid < kDigits) h[tid] = 0u;
    __syncthreads();
    uint32_t kv[kKSteps];
#pragma unroll
    for (int u = 0; u < kKSteps; ++u) {
        const int i = t * kSTile + u * kKThreads + tid;
        kv[u] = src[min(i, V - 1)];  // clamped: keys past V unused
    }
#pragma unroll
    for (int u = 0; u < kKSteps; ++u) {
        const int i = t * kSTile + u * kKThreads + tid;
        if (i < V) atomicAdd(&h[(kv[u] >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid < kDigits) split_row(a, row, T).cnt[t * kDigits + tid] = h[tid];
}

// 3b. Output position of each (digit, tile) group: digits in order, tiles in
//     order inside a digit (a stable pass). In place over the counts; thread
//     d walks its digit's counts down the tiles, 64 loads in flight, a wave's
//     loads of one tile on consecutive words.
__global__ __launch_bounds__(kSThreads) void fs_scan_kernel(DevArgs a, int T) {
    __shared__ uint32_t scan[kSWaves];
    constexpr int kB = 64;
    const int row = blockIdx.x, tid = threadIdx.x;
    uint32_t k;
    ge_sample_params p;
    if (!split_row_active(a, row, k, p)) return;
    uint32_t* c = split_row(a, row, T).cnt + tid;
    uint32_t total = 0;
    for (int t0 = 0; t0 < T; t0 += kB) {
        uint32_t v[kB];
#pragma unroll
        for (int u = 0; u < kB; ++u) v[u] = c[min(t0 + u, T - 1) * kDigits];
#pragma unroll
        for (int u = 0; u < kB; ++u) total += t0 + u < T ? v[u] : 0u;
    }
    uint32_t run = digit_excl_scan(total, scan, tid);
    for (int t0 = 0; t0 < T; t0 += kB) {
        uint32_t v[kB];
#pragma unroll
        for (int u = 0; u < kB; ++u) v[u] = c[min(t0 + u, T - 1) * kDigits];
#pragma unroll
        for (int u = 0; u < kB; ++u) {
            if (t0 + u < T) c[(t0 + u) * kDigits] = run;
            run += t0 + u < T ? v[u] : 0u;
        }
    }
}

// 3c. The stable scatter of tile t by the digit at `shift`: ranks among the
//     tile's keys of the same digit in position order (ballots per 64-key
//     step, per-wave LDS counters across steps), the keys grouped by digit in
//     LDS, each group stored at its output position (consecutive addresses).
//     With `fused` (a few rows), the tile computes its output bases from the
//     tiles' counts itself, as fs_scan_kernel would (which then is not
//     launched): every tile of a row reads the row's counts.
// (1024 threads, as fs_keys_kernel: threads tid < 256 hold the per-digit work)
__global__ __launch_bounds__(kKThreads) void fs_scatter_kernel(DevArgs a, int shift, int src_is_buf1, int fused) {
    constexpr int kKWaves = kKThreads / 64;
    __shared__ uint32_t staged[kSTile];
    __shared__ uint32_t wc[kKWaves][kDigits];
    __shared__ uint32_t toff[kDigits];
    __shared__ uint32_t gb[kDigits];
    __shared__ uint32_t scan[kKWaves];
    const int t = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    const int lane = __lane_id(), wave = tid >> 6;
    uint32_t k;
    ge_sample_params p;
    if (!split_row_active(a, row, k, p)) return;
    const int V = a.vocab, T = gridDim.x;
    uint32_t* b0 = reinterpret_cast<uint32_t*>(a.fo_aux) + static_cast<int64_t>(row) * a.fo_items_stride;
    uint32_t* b1 = a.fo_pre + static_cast<int64_t>(row) * a.fo_items_stride;
    const uint32_t* src = src_is_buf1 ? b1 : b0;
    uint32_t* dst = src_is_buf1 ? b0 : b1;
    uint32_t key[kKSteps];
#pragma unroll
    for (int u = 0; u < kKSteps; ++u) {
        const int i = t * kSTile + wave * (64 * kKSteps) + u * 64 + lane;
        key[u] = src[min(i, V - 1)];  // clamped: keys past V unused
    }
    for (int d = lane; d < kDigits; d += 64) wc[wave][d] = 0u;  // only this wave uses its row
    if (fused) {
        // digits before d over all tiles, then digit d in the tiles before t
        const uint32_t* c = split_row(a, row, T).cnt + min(tid, kDigits - 1);
        constexpr int kB = 16;
        uint32_t total = 0, part = 0;
        for (int t0 = 0; t0 < (tid < kDigits ? T : 0); t0 += kB) {
            uint32_t v[kB];
#pragma unroll
            for (int u = 0; u < kB; ++u) v[u] = c[min(t0 + u, T - 1) * kDigits];  // clamped
#pragma unroll
            for (int u = 0; u < kB; ++u) {
                const uint32_t x = t0 + u < T ? v[u] : 0u;
                total += x;
                part += t0 + u < t ? x : 0u;
            }
        }
        const uint32_t ex = digit_excl_scan(total, scan, tid);  // (scan[] is read again after a barrier)
        if (tid < kDigits) gb[tid] = ex + part;
    } else if (tid < kDigits) {
        gb[tid] = split_row(a, row, T).cnt[t * kDigits + tid];
    }
    const uint64_t below = (1ull << lane) - 1ull;
    uint32_t lr[kKSteps];
#pragma unroll
    for (int u = 0; u < kKSteps; ++u) {
        const int i = t * kSTile + wave * (64 * kKSteps) + u * 64 + lane;
        const bool act = i < V;
        const uint64_t am = __ballot(act);
        const uint32_t d = (key[u] >> shift) & 255u;
        const uint64_t mm = match_digit(d, am);
        lr[u] = 0u;
        if (act) {
            // lanes of one digit read the same counter, then all write the
            // same advanced value (in program order, so the next step reads it)
            const uint32_t c = wc[wave][d];
            lr[u] = c + static_cast<uint32_t>(__popcll(mm & below));
            wc[wave][d] = c + static_cast<uint32_t>(__popcll(mm));
        }
    }
    __syncthreads();
    uint32_t tot = 0;
    if (tid < kDigits) {
        for (int w = 0; w < kKWaves; ++w) {  // thread d: each wave's offset among the tile's keys of digit d
            const uint32_t c = wc[w][tid];
            wc[w][tid] = tot;
            tot += c;
        }
    }
    const uint32_t te = digit_excl_scan(tot, scan, tid);
    if (tid < kDigits) toff[tid] = te;
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kKSteps; ++u) {
        const int i = t * kSTile + wave * (64 * kKSteps) + u * 64 + lane;
        if (i < V) {
            const uint32_t d = (key[u] >> shift) & 255u;
            staged[toff[d] + wc[wave][d] + lr[u]] = key[u];
        }
    }
    __syncthreads();
    const int nt = min(kSTile, V - t * kSTile);
#pragma unroll
    for (int u = 0; u < kKSteps; ++u) {
        const int q = u * kKThreads + tid;
        if (q < nt) {
            const uint32_t kv = staged[q];
            const uint32_t d = (kv >> shift) & 255u;
            dst[gb[d] + static_cast<uint32_t>(q) - toff[d]] = kv;
        }
    }
}

// Item boundaries of the sorted keys: position i starts an item when i == 0
// or its key differs from position i - 1's.
__device__ __forceinline__ bool is_boundary(const uint32_t* s, int i, int V, uint32_t kv) {
    return i < V && (i == 0 || kv != s[i - 1]);
}

// 4a. Items starting in tile t.
__global__ __launch_bounds__(kKThreads) void fs_bounds_kernel(DevArgs a) {  // (1024 threads)
    constexpr int kKWaves = kKThreads / 64;
    __shared__ uint32_t red[kKWaves];
    const int t = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    uint32_t k;
    ge_sample_params p;
    if (!split_row_active(a, row, k, p)) return;
    const int V = a.vocab, T = gridDim.x;
    const uint32_t* s = reinterpret_cast<const uint32_t*>(a.fo_aux) + static_cast<int64_t>(row) * a.fo_items_stride;
    uint32_t n = 0;
#pragma unroll
    for (int u = 0; u < kKSteps; ++u) {
        const int i = t * kSTile + u * kKThreads + tid;
        const uint32_t kv = s[min(i, V - 1)];  // clamped: is_boundary checks i < V
        n += is_boundary(s, i, V, kv) ? 1u : 0u;
    }
    n = wave::readlane(wave::incl_add(n), 63);
    if (__lane_id() == 0) red[tid >> 6] = n;
    __syncthreads();
    if (tid == 0) {
        uint32_t c = 0;
        for (int w = 0; w < kKWaves; ++w) c += red[w];
        split_row(a, row, T).bc[t] = c;
    }
}

// 4b. Each item's first element into pre (buf1), in position order, and its
//     value into the high word of its items entry (4c adds the count); the
//     last tile also writes pre[G] = V.
__global__ __launch_bounds__(kKThreads) void fs_istart_kernel(DevArgs a) {  // (1024 threads)
    constexpr int kKWaves = kKThreads / 64;
    __shared__ uint32_t scan[kKWaves];
    __shared__ uint32_t base_s;
    const int t = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    const int lane = __lane_id(), wave = tid >> 6;
    uint32_t k;
    ge_sample_params p;
    if (!split_row_active(a, row, k, p)) return;
    const int V = a.vocab, T = gridDim.x;
    const SplitRow sr = split_row(a, row, T);
    const uint32_t* s = reinterpret_cast<const uint32_t*>(a.fo_aux) + static_cast<int64_t>(row) * a.fo_items_stride;
    uint32_t* istart = a.fo_pre + static_cast<int64_t>(row) * a.fo_items_stride;
    uint64_t* items = a.fo_items + static_cast<int64_t>(row) * a.fo_items_stride;
    if (wave == 0) {
        const uint32_t b = items_before(sr.bc, t);
        if (lane == 0) base_s = b;
    }
    // wave w owns positions [w * 256, (w + 1) * 256) of the tile
    uint32_t kv[kKSteps];
    bool bnd[kKSteps];
    uint32_t nb = 0;
#pragma unroll
    for (int u = 0; u < kKSteps; ++u) {
        const int i = t * kSTile + wave * (64 * kKSteps) + u * 64 + lane;
        kv[u] = s[min(i, V - 1)];  // clamped: is_boundary checks i < V
    }
#pragma unroll
    for (int u = 0; u < kKSteps; ++u) {
        const int i = t * kSTile + wave * (64 * kKSteps) + u * 64 + lane;
        bnd[u] = is_boundary(s, i, V, kv[u]);
        nb += static_cast<uint32_t>(__popcll(__ballot(bnd[u])));
    }
    if (lane == 0) scan[wave] = nb;
    __syncthreads();
    uint32_t j = base_s;
    for (int w = 0; w < wave; ++w) j += scan[w];
    const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
    for (int u = 0; u < kKSteps; ++u) {
        const int i = t * kSTile + wave * (64 * kKSteps) + u * 64 + lane;
        const uint64_t m = __ballot(bnd[u]);
        if (bnd[u]) {
            const uint32_t jj = j + static_cast<uint32_t>(__popcll(m & below));
            const uint32_t key = ~kv[u];
            istart[jj] = static_cast<uint32_t>(i);
            items[jj] = static_cast<uint64_t>(key == kKeyNaN ? 0x7fc00000u : f2u(key_value(key))) << 32;
        }
        j += static_cast<uint32_t>(__popcll(m));
    }
    if (t == T - 1 && tid == 0) {
        uint32_t c = base_s;
        for (int w = 0; w < kKWaves; ++w) c += scan[w];
        istart[c] = static_cast<uint32_t>(V);
    }
}

// 4c. The items that start in tile t: each one's count (from the next
//     item's first element) beside its value, its exp into aux
//     (generation.cpp:94-97: p = exp((l - max) * (1/T)), max the first
//     item's value), and the tile's part of the certificate of the top k's
//     double sum: the sum, the lowest set bit, any NaN. aux held the sorted
//     keys, which 4b was the last to read.
__global__ __launch_bounds__(kKThreads) void fs_exps_kernel(DevArgs a) {  // (1024 threads, as fs_keys_kernel)
    constexpr int kKWaves = kKThreads / 64;
    __shared__ uint32_t base_s;
    __shared__ double dred[kKWaves];
    __shared__ int ired[kKWaves];
    __shared__ uint32_t ured[kKWaves];
    const int t = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    const int lane = __lane_id(), wave = tid >> 6;
    uint32_t k;
    ge_sample_params p;
    if (!split_row_active(a, row, k, p)) return;
    const int T = gridDim.x;
    const SplitRow sr = split_row(a, row, T);
    const uint32_t* istart = a.fo_pre + static_cast<int64_t>(row) * a.fo_items_stride;
    uint64_t* items = a.fo_items + static_cast<int64_t>(row) * a.fo_items_stride;
    float* aux = a.fo_aux + static_cast<int64_t>(row) * a.fo_items_stride;
    if (wave == 0) {
        const uint32_t b = items_before(sr.bc, t);
        if (lane == 0) base_s = b;
    }
    __syncthreads();
    const float vmax = u2f(static_cast<uint32_t>(items[0] >> 32));
    const float inv_temp = 1.0f / p.temperature;
    const uint32_t j0 = base_s, nj = sr.bc[t];
    double S = 0.0;
    int minlsb = INT_MAX;
    bool nan = false;
    uint64_t itv[kKSteps];
    uint32_t stv[kKSteps], env[kKSteps];
    if (nj > 0u) {
#pragma unroll
        for (int u = 0; u < kKSteps; ++u) {  // nj <= kSTile; clamped indices, no conditional load
            const uint32_t q = min(static_cast<uint32_t>(u * kKThreads + tid), nj - 1u);
            itv[u] = items[j0 + q];
            stv[u] = istart[j0 + q];
            env[u] = istart[j0 + q + 1];
        }
    }
#pragma unroll
    for (int u = 0; u < kKSteps; ++u) {
        const uint32_t q = static_cast<uint32_t>(u * kKThreads + tid);
        if (q < nj) {
            const uint32_t n = env[u] - stv[u];
            const uint32_t vb = static_cast<uint32_t>(itv[u] >> 32);
            items[j0 + q] = (static_cast<uint64_t>(vb) << 32) | n;
            const float pe = expf_glibc((u2f(vb) - vmax) * inv_temp);
            aux[j0 + q] = pe;
            const uint32_t nk = top_k_count(stv[u], n, k);
            if (nk) {
                if (pe != pe) nan = true;
                else if (pe > 0.0f) {
                    minlsb = min(minlsb, lsb_exp(pe));
                    S += static_cast<double>(nk) * static_cast<double>(pe);
                }
            }
        }
    }
    S = wave::sum_f64(S);  // a certificate: exact whenever it certifies
    minlsb = wave::min_i32(minlsb);
    const uint32_t nanw = __ballot(nan) != 0ull ? 1u : 0u;
    if (lane == 0) {
        dred[wave] = S;
        ired[wave] = minlsb;
        ured[wave] = nanw;
    }
    __syncthreads();
    if (tid == 0) {
        double Sp = 0.0;
        int ml = INT_MAX;
        uint32_t nn = 0;
        for (int w = 0; w < kKWaves; ++w) {
            Sp += dred[w];
            ml = min(ml, ired[w]);
            nn |= ured[w];
        }
        const uint64_t sb = __builtin_bit_cast(uint64_t, Sp);
        uint32_t* pt = sr.part + 4 * t;
        pt[0] = static_cast<uint32_t>(sb);
        pt[1] = static_cast<uint32_t>(sb >> 32);
        pt[2] = static_cast<uint32_t>(ml);
        pt[3] = nn;
    }
}

// 4d. The row's meta words, as fo_sort_kernel writes them.
__global__ __launch_bounds__(64) void fs_meta_kernel(DevArgs a, int T) {
    const int row = blockIdx.x, lane = __lane_id();
    uint32_t k;
    ge_sample_params p;
    if (!split_row_active(a, row, k, p)) return;
    const SplitRow sr = split_row(a, row, T);
    double S = 0.0;
    int ml = INT_MAX;
    uint32_t nn = 0, G = 0;
    for (int t = lane; t < T; t += 64) {
        const uint32_t* pt = sr.part + 4 * t;
        S += __builtin_bit_cast(double, (static_cast<uint64_t>(pt[1]) << 32) | pt[0]);
        ml = min(ml, static_cast<int>(pt[2]));
        nn |= pt[3];
        G += sr.bc[t];
    }
    S = wave::sum_f64(S);
    ml = wave::min_i32(ml);
    nn = __ballot(nn != 0u) != 0ull ? 1u : 0u;
    G = wave::readlane(wave::incl_add(G), 63);
    if (lane == 0) {
        const uint64_t* items = a.fo_items + static_cast<int64_t>(row) * a.fo_items_stride;
        const uint32_t* istart = a.fo_pre + static_cast<int64_t>(row) * a.fo_items_stride;
        const bool last_nan = static_cast<uint32_t>(items[G - 1] >> 32) == 0x7fc00000u;
        uint32_t* meta = a.fo_meta + static_cast<int64_t>(row) * kMetaWords;
        const uint64_t sb = __builtin_bit_cast(uint64_t, S);
        meta[kMetaSumLo] = static_cast<uint32_t>(sb);
        meta[kMetaSumHi] = static_cast<uint32_t>(sb >> 32);
        meta[kMetaMinLsb] = static_cast<uint32_t>(ml);
        meta[kMetaAnyNan] = nn;
        meta[kMetaItems] = G;
        meta[kMetaExtras] = 0;
        meta[kMetaNan] = last_nan ? static_cast<uint32_t>(a.vocab) - istart[G - 1] : 0u;
        meta[kMetaStatus] = kStatusOk;
    }
}

// ---- kernel 2: probabilities, exact chains, token ----------------------------


// Item boundaries and addends: start(i) is the index of item i's first
// element, start(G) the element count. One view reads LDS copies (rows whose
// items fit), the other the global arrays; each is a single address space,
// so the compiler emits ds_read or global_load rather than flat loads.
struct LdsView {
    static constexpr int kPerLane = 2;  // mostly binade crossings: shorter steps
    const uint32_t* pre;
    const float* add;
    __device__ __forceinline__ uint32_t start(int i) const { return pre[i]; }
    __device__ __forceinline__ float addend(int i) const { return add[i]; }
};
struct GlobalView {
    static constexpr int kPerLane = 4;  // mostly plain steps: longer ones
    const uint32_t* pre;
    const float* add;
    __device__ __forceinline__ uint32_t start(int i) const { return pre[i]; }
    __device__ __forceinline__ float addend(int i) const { return add[i]; }
};

// Replays elements [cp.elem, L) of the accumulation described by the items,
// with one wave, 64 items per step. kDesc: c -= a, stopping at the first
// element with c <= a; else s += a, stopping at the first element whose sum
// is >= thr (NaN: never). Returns true on an event with cp at the event
// element; otherwise false with cp.elem == L and cp.item holding element L-1.
// Requires cp.elem < L <= start(G).
//
// Each lane takes one item: its increment in the current binade (count x
// whole ulps) is scanned across the wave; lanes before the first one that
// would leave the binade, tie or reach the threshold are applied at once,
// and that lane runs the closed form of chain_math.h.
template <typename Acc, bool kDesc, typename View>
__device__ bool wave_chain(const View& iv, int G, ChainPos& cp, uint32_t L, double& s, double thr) {
    constexpr int P = chain::AccTraits<Acc>::P;
    constexpr bool kF32 = P == 24;
    const int lane = __lane_id();
    while (cp.elem < L && cp.item < G) {
        const int i = cp.item + lane;
        uint32_t nt = 0, lo_e = 0;
        double av = 0.0;
        if (i < G) {
            const uint32_t st = iv.start(i);
            const uint32_t en = iv.start(i + 1);
            lo_e = max(st, cp.elem);
            const uint32_t hi_e = min(en, L);
            nt = hi_e > lo_e ? hi_e - lo_e : 0u;
            av = static_cast<double>(iv.addend(i));
        }
        const chain::Binade b = chain::binade_of<Acc>(s);
        const chain::Step st = chain::step_of<Acc>(b, av);
        bool ev = false;
        double incl_d = 0.0;
        uint64_t incl_u = 0;
        if (kF32) {
            // room in a float binade < 2^24: capping each lane at 2^40 keeps
            // every partial sum exact in double and every exit detected
            double tot = 0.0;
            if (nt && !st.big) tot = min(static_cast<double>(nt) * static_cast<double>(st.D), 1099511627776.0);
            incl_d = wave_incl_f64(tot);
            const double m = static_cast<double>(b.m);
            if (nt) {
                if (kDesc) {
                    ev = st.big || st.tie || m - incl_d < static_cast<double>(b.lo);
                } else {
                    double tm = 1e300;
                    if (thr == thr) {
                        if (!(thr > 0.0)) tm = 0.0;
                        else if (thr < std::ldexp(1.0, b.uexp + P))
                            tm = static_cast<double>(chain::threshold_m(thr, b.uexp));
                    }
                    ev = st.big || st.tie || m + incl_d > static_cast<double>(b.hi) || m + incl_d >= tm;
                }
            }
        } else {
            const uint64_t tot = (nt && !st.big) ? sat_mul(nt, st.D) : 0;
            incl_u = wave_incl_u64_sat(tot);
            if (nt) {
                if (kDesc) {
                    ev = st.big || st.tie || b.m < b.lo + incl_u;
                } else {
                    uint64_t tm = chain::kNone;
                    if (thr == thr) {
                        if (!(thr > 0.0)) tm = 0;
                        else if (thr < std::ldexp(1.0, b.uexp + P)) tm = chain::threshold_m(thr, b.uexp);
                    }
                    ev = st.big || st.tie || b.m + incl_u > b.hi || b.m + incl_u >= tm;
                }
            }
        }
        auto applied = [&](int upto) -> uint64_t {  // ulps added by lanes < upto
            if (upto == 0) return 0;
            return kF32 ? static_cast<uint64_t>(rld(incl_d, upto - 1)) : rl64(incl_u, upto - 1);
        };
        const uint64_t evmask = __ballot(ev);
        if (evmask == 0) {
            const uint64_t total = applied(64);
            const uint64_t m2 = kDesc ? b.m - total : b.m + total;
            s = std::ldexp(static_cast<double>(m2), b.uexp);
            const int next = cp.item + 64;
            const uint32_t tile_end = next < G ? iv.start(next) : iv.start(G);
            if (tile_end >= L) {  // the last element lies in this tile
                const uint64_t lm = __ballot(nt && lo_e + nt == L);
                cp.item += static_cast<int>(__builtin_ctzll(lm));
                cp.elem = L;
                return false;
            }
            cp.elem = tile_end;
            cp.item = next;
            continue;
        }
        const int f = static_cast<int>(__builtin_ctzll(evmask));
        const uint64_t before = applied(f);
        const uint64_t m2 = kDesc ? b.m - before : b.m + before;
        s = std::ldexp(static_cast<double>(m2), b.uexp);
        cp.elem = rl32(lo_e, f);
        const uint32_t nf = rl32(nt, f);
        const double af = rld(av, f);
        bool evt = false;
        const uint64_t used = kDesc ? chain::desc_run<Acc>(s, af, nf, evt)
                                    : chain::asc_run<Acc>(s, af, nf, thr, evt);
        cp.item += f;
        if (evt) {
            cp.elem += static_cast<uint32_t>(kDesc ? used : used - 1);
            return true;
        }
        cp.elem += nf;
        if (cp.elem >= L) return false;
        cp.item += 1;
    }
    return false;
}

// Index of the item holding element x (pre[] strictly increasing, pre[0] = 0),
// by a 64-way search with one wave.
__device__ int wave_find_item(const uint32_t* pre, int G, uint32_t x) {
    const int lane = __lane_id();
    int lo = 0, hi = G;  // answer in [lo, hi)
    while (hi - lo > 1) {
        const int span = hi - lo;
        const int step = (span + 63) / 64;
        const int probe = lo + lane * step;
        const bool le = probe < hi && pre[probe] <= x;
        const uint64_t m = __ballot(le);
        const int last = 63 - static_cast<int>(__builtin_clzll(m));  // lane 0 always qualifies
        lo = lo + last * step;
        hi = min(hi, lo + step);
    }
    return lo;
}

constexpr int kDThreads = 512;
constexpr int kDWaves = kDThreads / 64;
constexpr int kStage = 8192;  // items whose count and probability are staged in LDS

// bf16 rows: the token scan's speculative batch counts (decide step 5s).
constexpr int kSpecGroups = 8;           // candidate groups, at most
constexpr int kSpecBefore = 2;           // items picked: the crossing item - 2 ..
constexpr int kSpecAfter = 3;            //   .. the crossing item + 3
constexpr int kSpecBatch = kDThreads * 32;  // tokens per bf16 token-scan batch
constexpr int kSpecBatches = 32;         // batches counted (rows up to 32 x 16384 tokens)
constexpr int kSpecBlock = 64 * 32;      // tokens a counting wave takes per round
constexpr uint32_t kSpecWaves = 0xFEu;   // the counting waves (wave 1 picks the groups)
constexpr int kSpecCounters = __builtin_popcount(kSpecWaves);
static_assert(kSpecBefore + 1 + kSpecAfter <= kSpecGroups, "the picked items fit the candidates");
static_assert((kSpecWaves & 3u) == 2u, "wave 0 draws, wave 1 picks and counts");
static_assert(kSpecBatch % kSpecBlock == 0, "a counting round lies in one batch");
// bf16 rows: the top-p chain's skip table (decide step 5t), in segments of one
// wave-chain step over LDS items, built by waves 2-7.
constexpr int kSkipSeg = 64 * LdsView::kPerLane;
constexpr int kSkipSegs = kStage / kSkipSeg;
constexpr int kSkipBuilders = 6;
static_assert((kSpecWaves & 0xFCu) == 0xFCu && kDWaves == 8, "waves 2-7 build the skip table");

struct DecideShared {
    union {
        struct {
            uint32_t pre[kStage + 1];  // item boundaries (elements before each item)
            float add[kStage];         // per-item probability
        } st;
        uint32_t gx_ids[kFoExtrasCap];  // penalised tokens of the selected value, ascending
    };
    bchain::Shared<kDWaves> bc;  // block chains (sorted rows)
    double dred[kDWaves];
    int ired[kDWaves];
    uint32_t ured[kDWaves];
    uint32_t scan[kDWaves];
    uint32_t tscan[2][kDWaves];  // the token scan's wave sums, by batch parity
    double den;
    uint32_t pos, group_rank, group_total, forward, gx_count;
    uint32_t blo, bhi, nan_group, near, gkey;
    int32_t token;
    int item;
    // bf16 rows: the token scan's speculative batch counts (see the decide
    // kernel's step 6s), made by waves 1.. while wave 0 draws.
    uint32_t spec_cnt[kSpecGroups][kSpecBatches];
    uint32_t spec_key[kSpecGroups], spec_blo[kSpecGroups], spec_bhi[kSpecGroups];
    uint32_t skip_tot[kSkipSegs];               // the top-p chain's skip table
    uint32_t skip_flags[(kSkipSegs + 31) / 32];
    uint32_t skip_built;                        // builder waves done
    uint32_t spec_bdone[kSpecBatches];  // blocks of each batch counted
    uint32_t spec_ulo, spec_uhi;  // the candidates' bins lie in [spec_ulo, spec_uhi]
    uint32_t spec_n;              // candidate groups (0: none)
    uint32_t spec_fwd;            // the predicted scan direction
    uint32_t spec_nbat;           // batches to count, from that direction's end
    uint32_t spec_ready;          // wave 1 has written the candidates
    uint32_t spec_stop;           // wave 0 has drawn: the count pass stops
};

// ---- the double denominator's tile maps (sorted rows) ----------------------
//
// When a sorted row's double sum over its top k does not certify (its terms
// span more than the 53 bits above their lowest set bit), the reference's
// sequential sum (generation.cpp:97) has to be replayed. Inside one binade
// of the accumulator a run of elements is a parity map (chain_math.h), and
// maps compose. So the items are cut into tiles of block_chain's size, each
// in kMapSub parts, and a workgroup per part composes the part's map for the
// top kMapBins binades the sum can be in (fo_denmap_kernel, before
// fo_decide_kernel). The decide kernel then applies one map per part; from a
// part whose map leaves the accumulator's binade (or whose binade has no
// map) it replays the rest of the tile with block_chain. The maps live in
// the row's share of the tile area (fo_tiles), which the many-workgroup sort
// has finished with by then.
constexpr int kMapTile = kDThreads * bchain::kPer;  // items per tile: block_chain's tile
constexpr int kMapSub = 4;                           // parts per tile, one workgroup each
constexpr int kMapSubItems = kMapTile / kMapSub;
constexpr int kMapGroup = 256;                       // threads per binade slot
constexpr int kMapPer = kMapSubItems / kMapGroup;    // items per thread
constexpr int kMapBins = 3;                          // binades bhi - 2 .. bhi (bhi: the sum's, plus one)
constexpr int kMapRowGroups = 16;                    // grid rows: row r is served by grid row r % 16
constexpr int kMapPartWords = kMapBins * 4;          // 4 u32 (e, o) per binade
using DMap = chain::ParityMap<uint64_t>;
constexpr uint64_t kMapCap = bchain::F64Acc::kCap;
static_assert(kMapSubItems % kMapGroup == 0, "whole items per thread");
constexpr int kMapThreads = kMapGroup * kMapBins;   // the slots side by side, one group each
static_assert(kMapTile == 4096 && kMapSub * kMapPartWords <= 256 + 1 + 4, "a tile's maps fit its share of the tile area");

// Words of one row's maps.
__host__ __device__ constexpr int64_t map_row_words(int vocab) {
    return static_cast<int64_t>((vocab + kMapTile - 1) / kMapTile) * kMapSub * kMapPartWords;
}

// Whether a sorted row's denominator needs no replay: its certificate (the
// parallel sum S, the lowest set bit of every term, NaN) from the meta words
// (a NaN term makes the sum NaN: no replay either).
__device__ __forceinline__ bool den_certified(const uint32_t* meta, double& S) {
    S = __builtin_bit_cast(double, (static_cast<uint64_t>(meta[kMetaSumHi]) << 32) | meta[kMetaSumLo]);
    const int minlsb = static_cast<int>(meta[kMetaMinLsb]);
    const bool nan = meta[kMetaAnyNan] != 0u;
    return nan || S == 0.0 || minlsb >= exp_of(S) - 51;
}

// The largest binade the sequential sum can reach: that of the parallel sum
// S plus one (the two differ by far less than a binade).
__device__ __forceinline__ int den_top_binade(double S) { return exp_of(S) + 1; }

// Whether part `part` (tile * kMapSub + p) of row `row` needs its maps: a
// sorted row of this pass whose sum does not certify, with items in the part.
__device__ __forceinline__ bool map_part_needed(const DevArgs& a, int row, int part) {
    uint32_t k;
    if (!full_order_row(params_of(a, row), a.vocab, k) || row_done(a, row) || k <= 1u) return false;
    const uint32_t* meta = a.fo_meta + static_cast<int64_t>(row) * kMetaWords;
    if (meta[kMetaStatus] != (a.fo_fallback ? kStatusFallback : kStatusOk)) return false;
    if (part * kMapSubItems >= static_cast<int>(meta[kMetaItems])) return false;
    double S;
    return !den_certified(meta, S);
}

// The maps of one part (block-uniform): its items' elements in [1, k)
// (element 0, the maximum's term, starts the sum), composed for each binade
// 2^b, b in [bhi - 2, bhi], that the sum can be in while the part is added;
// a binade below a lower bound of the sum before the part gets a saturated
// map (the decide kernel then replays).
__device__ __forceinline__ void map_part(const DevArgs& a, int row, int part, uint64_t (&wmap)[2][kMapThreads / 64]) {
    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int wave = tid >> 6;
    const int V = a.vocab;
    uint32_t k = 0;
    (void)full_order_row(params_of(a, row), V, k);
    const uint32_t* meta = a.fo_meta + static_cast<int64_t>(row) * kMetaWords;
    const int G = static_cast<int>(meta[kMetaItems]);
    double S;
    (void)den_certified(meta, S);
    const int i0 = part * kMapSubItems;
    const uint32_t* pre = a.fo_pre + static_cast<int64_t>(row) * a.fo_items_stride;
    const float* aux = a.fo_aux + static_cast<int64_t>(row) * a.fo_items_stride;
    uint32_t* out = a.fo_tiles + static_cast<int64_t>(row) * fo_tile_words(fo_split_tiles(V)) +
                    static_cast<int64_t>(part) * kMapPartWords;
    // Lower bounds of the sum before this part (terms only fall along the
    // list): its elements times the part's first term; and the whole sum
    // less every later element at that term (S within 2^-30 of the
    // sequential sum, with room to spare).
    const uint32_t e_before = min(max(pre[i0], 1u), k);
    const double t0 = static_cast<double>(aux[i0]);
    const double lb1 = static_cast<double>(e_before) * t0;
    const double lb2 = S * (1.0 - 0x1p-30) - static_cast<double>(k - e_before) * t0 * (1.0 + 0x1p-30);
    const double lb = max(lb1, lb2);
    const int blo = lb >= 1.0 ? exp_of(lb) : 0;
    const int bhi = den_top_binade(S);
    // Each group of kMapGroup threads composes one slot's map (the slots
    // side by side: one wave per SIMD left their dependent steps
    // latency-bound). This thread's items (clamped loads: items past G hold
    // no element).
    const int slot = tid / kMapGroup;
    const int gt = tid % kMapGroup;
    constexpr int kGW = kMapGroup / 64;  // waves per group
    uint32_t pb[kMapPer + 1];
    uint32_t ab[kMapPer];
    const int ib = i0 + gt * kMapPer;
#pragma unroll
    for (int j = 0; j <= kMapPer; ++j) pb[j] = min(pre[min(ib + j, G)], k);
#pragma unroll
    for (int j = 0; j < kMapPer; ++j) ab[j] = f2u(aux[min(ib + j, G - 1)]);
    const int b = bhi - (kMapBins - 1) + slot;
    const bool live = b >= blo && b >= 0;  // (uniform in the group)
    if (live) {
        const int uexp = b - 52;
        DMap f{0, 0};
#pragma unroll
        for (int j = 0; j < kMapPer; ++j) {
            const uint32_t lo = max(pb[j], 1u);
            const uint32_t nt = pb[j + 1] > lo ? pb[j + 1] - lo : 0u;
            uint64_t D;
            bool tie, odd0, big;
            chain::step_bits64(ab[j], uexp, D, tie, odd0, big);
            f = chain::compose<uint64_t, kMapCap>(f, chain::run_map<uint64_t, kMapCap>(nt, D, tie, odd0, big));
        }
        const DMap x = map_wave_excl<uint64_t, kMapCap>(f);
        if (lane == 63) {
            const DMap wt = chain::compose<uint64_t, kMapCap>(x, f);
            wmap[0][wave] = wt.e;
            wmap[1][wave] = wt.o;
        }
    }
    __syncthreads();
    if (gt == 0) {
        DMap tot{kMapCap, kMapCap};
        if (live) {
            tot = DMap{0, 0};
#pragma unroll
            for (int w = 0; w < kGW; ++w)
                tot = chain::compose<uint64_t, kMapCap>(tot, DMap{wmap[0][slot * kGW + w], wmap[1][slot * kGW + w]});
        }
        out[4 * slot + 0] = static_cast<uint32_t>(tot.e);
        out[4 * slot + 1] = static_cast<uint32_t>(tot.e >> 32);
        out[4 * slot + 2] = static_cast<uint32_t>(tot.o);
        out[4 * slot + 3] = static_cast<uint32_t>(tot.o >> 32);
    }
    __syncthreads();  // wmap is read before the next part writes it
}

__global__ __launch_bounds__(kMapThreads) void fo_denmap_kernel(DevArgs a) {
    __shared__ uint64_t wmap[2][kMapThreads / 64];
    __shared__ uint64_t need_rows;
    const int lane = __lane_id();
    const int part = static_cast<int>(blockIdx.x);
    if ((threadIdx.x >> 6) == 0) {
        const int r = static_cast<int>(blockIdx.y) + lane * static_cast<int>(gridDim.y);
        const uint64_t m = __ballot(r < a.rows && map_part_needed(a, r, part));
        if (lane == 0) need_rows = m;
    }
    __syncthreads();
    uint64_t todo = need_rows;
    while (todo) {
        const int j = __ffsll(static_cast<unsigned long long>(todo)) - 1;
        todo &= todo - 1ull;
        map_part(a, static_cast<int>(blockIdx.y) + j * static_cast<int>(gridDim.y), part, wmap);
    }
}

// The sequential double sum over elements [1, k) of a sorted row, from s =
// the first term: the parts' maps (fo_denmap_kernel) for the accumulator's
// binade are composed 64 parts at a time by a wave scan, which finds the
// first part that would leave the binade (or whose binade has no map); the
// rest of that part's tile is replayed exactly by block_chain, and the scan
// resumes at the next tile. The parts' maps and end elements are first
// staged in `stage` (LDS, ntiles * kMapSub * (kMapPartWords + 1) + 8
// words). Block-uniform (block_chain holds barriers). Kept out of line:
// inlined, it changed the decide kernel's code for every row (certified rows
// 26 µs slower per launch of 256 C4-f32 rows).
__device__ __attribute__((noinline)) double den_by_maps(const DevArgs& a, int row, const uint32_t* pre, const float* aux,
                                                        int G, uint32_t k, double s2, double S, uint32_t* stage,
                                                        bchain::Shared<kDThreads / 64>& bc) {
    const int tid = static_cast<int>(threadIdx.x);
    const int lane = __lane_id();
    const uint32_t* maps = a.fo_tiles + static_cast<int64_t>(row) * fo_tile_words(fo_split_tiles(a.vocab));
    const int ntiles = (G + kMapTile - 1) / kMapTile;
    const int nparts = ntiles * kMapSub;
    uint32_t* pend = stage + nparts * kMapPartWords;  // end element of each part (clipped to k)
    uint64_t* res = reinterpret_cast<uint64_t*>(stage + ((nparts * (kMapPartWords + 1) + 1) & ~1));  // scan result
    for (int i = tid; i < nparts * kMapPartWords; i += kDThreads) stage[i] = maps[i];
    for (int i = tid; i < nparts; i += kDThreads) pend[i] = min(pre[min((i + 1) * kMapSubItems, G)], k);
    __syncthreads();
    const int bhi = den_top_binade(S);
    auto start_elem = [&](int q) { return q == 0 ? 1u : pend[q - 1]; };
    int p = 0;  // next part; the sum holds every element before start_elem(p)
    while (p < nparts && start_elem(p) < k) {
        const bchain::F64Acc::Bin bn = bchain::F64Acc::binade(s2, __builtin_nan(""));
        const int slot = bn.uexp + 52 - (bhi - (kMapBins - 1));
        int crossing = p;  // first part not covered by a map
        bool found = true;  // a part at `crossing` needs the replay (else: 64 parts applied)
        if (slot >= 0 && slot < kMapBins) {
            if (tid < 64) {
                // Lane l: part p + l's map (identity past the last part);
                // the scan gives each lane the composition of the parts
                // before it, and the first lane whose part takes m past the
                // binade's top is the crossing.
                const int q = p + lane;
                DMap f{0, 0};
                if (q < nparts && start_elem(q) < k) {  // (parts past the last element have no maps written)
                    const uint32_t* w = stage + q * kMapPartWords + 4 * slot;
                    f = DMap{(static_cast<uint64_t>(w[1]) << 32) | w[0], (static_cast<uint64_t>(w[3]) << 32) | w[2]};
                }
                const DMap x = map_wave_excl<uint64_t, kMapCap>(f);
                const uint64_t rx = chain::apply_from(x, bn.m);  // parts before lane l
                const uint64_t ri = chain::apply_from(chain::compose<uint64_t, kMapCap>(x, f), bn.m);
                const uint64_t out = __ballot(q < nparts && start_elem(q) < k && bn.m + ri > bn.hi);
                const int n = min(64, nparts - p);
                const int first = out ? __ffsll(static_cast<unsigned long long>(out)) - 1 : n;
                const uint64_t rb = first < 64 ? wave::readlane64(rx, first) : wave::readlane64(ri, 63);
                if (lane == 0) {
                    res[0] = static_cast<uint64_t>(p + first);
                    res[1] = rb;
                    res[2] = out ? 1ull : 0ull;
                }
            }
            __syncthreads();
            crossing = static_cast<int>(res[0]);
            found = res[2] != 0ull;
            s2 = bchain::F64Acc::rebuild(s2, bn, bn.m + res[1]);
            __syncthreads();  // res is read before the next round writes it
        }
        if (crossing >= nparts || start_elem(crossing) >= k) break;
        if (!found) {
            p = crossing;  // 64 parts applied, none left the binade
            continue;
        }
        // Replay from part `crossing` to the end of its tile.
        const int t = crossing / kMapSub;
        const uint32_t tend = pend[t * kMapSub + kMapSub - 1];
        ChainPos cp{crossing * kMapSubItems, start_elem(crossing)};
        if (tend > cp.elem)
            (void)bchain::block_chain<bchain::F64Acc, false, kDThreads>(pre, aux, 1.0f, G, cp, tend, s2,
                                                                       __builtin_nan(""), bc);
        p = (t + 1) * kMapSub;
    }
    __syncthreads();  // every thread has read the staged maps before the caller reuses the area
    return s2;
}

template <typename T, typename Op>
__device__ __forceinline__ T wave_reduce(T v, Op op) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v = op(v, __shfl_xor(v, d, 64));
    return v;
}

// Block-wide exclusive scan for kDThreads threads.
__device__ __forceinline__ uint32_t dblock_excl_scan(uint32_t v, uint32_t* scratch, uint32_t& total) {
    const int lane = __lane_id();
    const int wave = threadIdx.x >> 6;
    const uint32_t incl = wave_incl_u32(v);
    if (lane == 63) scratch[wave] = incl;
    __syncthreads();
    uint32_t before = 0;
    total = 0;
#pragma unroll
    for (int w = 0; w < kDWaves; ++w) {
        const uint32_t x = scratch[w];
        if (w < wave) before += x;
        total += x;
    }
    __syncthreads();
    return before + incl - v;
}

// First index in [lo, hi) whose predicate is false, for a predicate that is
// true on a prefix; 64-way search with one wave.
template <typename Pred>
__device__ uint32_t wave_partition_point(uint32_t lo, uint32_t hi, Pred pred) {
    const int lane = __lane_id();
    while (hi > lo) {
        const uint32_t step = (hi - lo + 63) / 64;
        const uint32_t probe = lo + static_cast<uint32_t>(lane) * step;
        const uint64_t m = __ballot(probe < hi && pred(probe));
        if (m == 0) break;  // pred(lo) is false
        const int last = 63 - static_cast<int>(__builtin_clzll(m));
        lo = lo + static_cast<uint32_t>(last) * step + 1;
        hi = min(hi, lo - 1 + step);
    }
    return lo;
}

// The same partition point, searched first in the 64 keys from w0 = c - 32
// (clamped into [lo, hi)) around a guess c: one round when the boundary lies
// there, else the search above over the side it lies on. Exact whatever the
// guess (pred is monotone: true, then false).
template <typename Pred>
__device__ uint32_t wave_partition_point_near(uint32_t lo, uint32_t hi, uint32_t c, Pred pred) {
    if (hi <= lo) return lo;
    uint32_t w0 = c > lo + 32u ? c - 32u : lo;
    w0 = min(w0, hi - 1u);
    const uint32_t wn = min(64u, hi - w0);  // keys of the window inside [lo, hi)
    const uint32_t probe = w0 + static_cast<uint32_t>(__lane_id());
    const uint64_t m = __ballot(probe - w0 < wn && pred(probe));
    if (m & 1ull) {  // pred(w0): the boundary is in the window or after it
        const uint32_t n = static_cast<uint32_t>(__popcll(m));
        if (n < wn) return w0 + n;
        return w0 + wn >= hi ? hi : wave_partition_point(w0 + wn, hi, pred);
    }
    return w0 == lo ? lo : wave_partition_point(lo, w0, pred);
}

// T: the logits' type. kSorted: the items come from the sort kernel (every
// token in them, penalised ones at their final values; raw keys are f32
// order keys), else from the bf16 histogram (penalised tokens in the
// extras, raw keys are bf16 bins).
// bf16 rows run two workgroups per CU (8 waves each: 4 per SIMD, at most 128
// VGPRs); sorted rows one.
template <typename T, bool kSorted>
__global__ __launch_bounds__(kDThreads, kSorted ? 2 : 4) void fo_decide_kernel(DevArgs a) {
    constexpr bool kF32 = kSorted;
    __shared__ DecideShared sh;
    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int wave = tid >> 6;
    const int row = blockIdx.x;
    const int V = a.vocab;
    const ge_sample_params p = params_of(a, row);
    uint32_t k;
    if (!full_order_row(p, V, k)) return;
    if (row_done(a, row)) {  // finished by an earlier call: the first kernel skipped it too
        if (tid == 0 && !a.fo_fallback) skipped_row(a, row);
        return;
    }
    if (a.fo_fallback && a.fo_meta[static_cast<int64_t>(row) * kMetaWords + kMetaStatus] != kStatusFallback) return;

    const int32_t* hist;
    int H;
    history_of(a, row, hist, H);
    const bool pen = H > 0 && !(p.repetition_penalty == 1.0f);
    uint32_t* bitmap = a.fo_bitmap + static_cast<int64_t>(row) * a.fo_bitmap_words;
    const uint32_t* meta = a.fo_meta + static_cast<int64_t>(row) * kMetaWords;
    // The bitmap is all zero again after every call. It is cleared from the
    // history before the token is appended: with a device ring the history
    // IS the ring, and once it is full the new token overwrites the oldest
    // id, whose bit must be cleared from the id read here, not from the token.
    auto finish = [&](int32_t token, float prob, int32_t flags) {
        if (pen) {
            __syncthreads();
            for (int i = tid; i < H; i += kDThreads) {
                const int32_t id = hist[i];
                if (id >= 0 && id < V) bitmap[id >> 5] = 0u;
            }
            __syncthreads();  // every read of the ring precedes the append below
        }
        if (tid == 0) emit_row(a, row, token, prob, flags);
    };
    if (meta[kMetaStatus] != (a.fo_fallback ? kStatusFallback : kStatusOk)) {
        // Too many unique penalised ids for the extras: the fallback pass
        // re-samples the row (the caller launches it whenever a history may
        // be that long).
        finish(-1, 0.0f, GE_FLAG_UNSUPPORTED);
        return;
    }
    const int G = static_cast<int>(meta[kMetaItems]);
    const uint64_t* items = a.fo_items + static_cast<int64_t>(row) * a.fo_items_stride;
    float* aux = a.fo_aux + static_cast<int64_t>(row) * a.fo_items_stride;
    uint32_t* pre = a.fo_pre + static_cast<int64_t>(row) * a.fo_items_stride;
    const uint64_t* extras = a.fo_extras + static_cast<int64_t>(row) * a.fo_extras_cap;
    const uint32_t E = meta[kMetaExtras];

    // 4a. Per item: elements before it, exp, certificate of the double sum;
    //     512 items per round. generation.cpp:94-97: p = exp((l - max) * (1/T)).
    const float inv_temp = 1.0f / p.temperature;
    const float vmax = u2f(static_cast<uint32_t>(items[0] >> 32));
    const float p0 = expf_glibc((vmax - vmax) * inv_temp);
    double S = 0.0;
    int minlsb = INT_MAX;
    bool nan = false;
    uint32_t run_base = 0;
    if constexpr (kSorted) {
        // The sort kernel wrote each item's exp to aux (and every item's first
        // element to pre, pre[G] = V) and the certificate of their double sum
        // over the top k to the row's meta words.
        if (tid == 0) {
            S = __builtin_bit_cast(double, (static_cast<uint64_t>(meta[kMetaSumHi]) << 32) | meta[kMetaSumLo]);
            minlsb = static_cast<int>(meta[kMetaMinLsb]);
            nan = meta[kMetaAnyNan] != 0u;
        }
    }
    // (clamped prefetch: a masked load would wait for every load in flight)
    uint64_t it_next = !kSorted ? items[min(tid, G - 1)] : 0ull;
    for (int r0 = 0; r0 < (kSorted ? 0 : G); r0 += kDThreads) {
        const int i = r0 + tid;
        // the next round's item loads while this one is scanned; lanes past
        // G take 0 (an empty item) whatever the clamped load returned
        const uint64_t it = i < G ? it_next : 0ull;
        it_next = items[min(i + kDThreads, G - 1)];
        const uint32_t n = static_cast<uint32_t>(it);
        uint32_t tot;
        const uint32_t pi = run_base + dblock_excl_scan(n, sh.scan, tot);
        run_base += tot;
        if (i < G) {
            pre[i] = pi;
            if (i <= kStage) sh.st.pre[i] = pi;
            const uint32_t nk = top_k_count(pi, n, k);
            const float pe = expf_glibc((u2f(static_cast<uint32_t>(it >> 32)) - vmax) * inv_temp);
            aux[i] = pe;
            if (i < kStage) sh.st.add[i] = pe;
            if (nk) {
                if (pe != pe) nan = true;
                else if (pe > 0.0f) {
                    minlsb = min(minlsb, lsb_exp(pe));
                    S += static_cast<double>(nk) * static_cast<double>(pe);
                }
            }
        }
    }
    if (!kSorted && tid == 0) {
        pre[G] = run_base;
        if (G <= kStage) sh.st.pre[G] = run_base;
    }
    S = wave_reduce(S, [](double x, double y) { return x + y; });
    minlsb = wave_reduce(minlsb, [](int x, int y) { return min(x, y); });
    const uint32_t nanw = __ballot(nan) != 0;
    if (lane == 0) {
        sh.dred[wave] = S;
        sh.ired[wave] = minlsb;
        sh.ured[wave] = nanw;
    }
    __syncthreads();
    double Sp = 0.0;
    int ml = INT_MAX;
    uint32_t nn = 0;
    for (int w = 0; w < kDWaves; ++w) {
        Sp += sh.dred[w];
        ml = min(ml, sh.ired[w]);
        nn |= sh.ured[w];
    }
    const bool any_nan = nn != 0;
    // Every term is a multiple of 2^minlsb; if the sum needs at most 53 bits
    // above that, every partial sum in every order is exact, so the parallel
    // sum equals the reference's sequential one (generation.cpp:97).
    const bool certified = !any_nan && (Sp == 0.0 || ml >= exp_of(Sp) - 51);
    if constexpr (kSorted) {
        // up to V single-token items: the whole block replays the sum
        double den = Sp;
        if (any_nan) {
            den = __builtin_nan("");
        } else if (!certified) {
            ChainPos cp{0, 1};
            double s2 = static_cast<double>(p0);
            if (k > 1 && a.fo_maps) {
                s2 = den_by_maps(a, row, pre, aux, G, k, s2, Sp, sh.gx_ids, sh.bc);
            } else if (k > 1) {
                bchain::block_chain<bchain::F64Acc, false, kDThreads>(pre, aux, 1.0f, G, cp, k, s2, __builtin_nan(""), sh.bc);
            }
            den = s2;
        }
        if (tid == 0) sh.den = den;
    } else if (wave == 0) {
        double den = Sp;
        if (any_nan) {
            den = __builtin_nan("");
        } else if (!certified) {
            ChainPos cp{0, 1};
            double s2 = static_cast<double>(p0);
            if (k > 1) {
                if (G <= kStage) wave_chain<double, false>(LdsView{sh.st.pre, sh.st.add}, G, cp, k, s2, __builtin_nan(""));
                else wave_chain<double, false>(GlobalView{pre, aux}, G, cp, k, s2, __builtin_nan(""));
            }
            den = s2;
        }
        if (lane == 0) sh.den = den;
    }
    __syncthreads();

    // 4b. generation.cpp:98-101: inv = float(1/den); probs *= inv.
    //     generation.cpp:104: minimum = probs[0] * min_p.
    const float inv = static_cast<float>(1.0 / sh.den);
    const float q0 = p0 * inv;
    const float minimum = q0 * p.min_p;
    int first_low = INT_MAX;
    if constexpr (kSorted) {
        // The probabilities stay unscaled in aux: every reader takes
        // aux[i] * inv, the float operation a scaling pass would store. With
        // no NaN they are non-increasing (sorted values, monotone expf), so
        // the min-p cut (generation.cpp:106-108: the first element e >= 1
        // with p_e < minimum, within the top k) is a search, not a pass.
        if (!any_nan && minimum > 0.0f && G > 1) {
            const uint32_t pp = wave_partition_point(1u, static_cast<uint32_t>(G),
                                                     [&](uint32_t i) { return !(aux[i] * inv < minimum); });
            if (pp < static_cast<uint32_t>(G) && pre[pp] < k) first_low = static_cast<int>(pp);
        }
    } else {
        for (int i = tid; i < G; i += kDThreads) {  // this thread staged item i in 4a
            const float q = (i < kStage ? sh.st.add[i] : aux[i]) * inv;
            aux[i] = q;
            if (i < kStage) sh.st.add[i] = q;
            if (i >= 1 && first_low == INT_MAX && q < minimum && (i <= kStage ? sh.st.pre[i] : pre[i]) < k) first_low = i;
        }
    }
    first_low = wave_reduce(first_low, [](int x, int y) { return min(x, y); });
    __syncthreads();  // every reader of sh.ired above is done
    if (lane == 0) sh.ired[wave] = first_low;
    // step 5s (bf16 rows): the counts start at zero, nothing published
    const bool spec_on = !kSorted && !any_nan && V <= kSpecBatches * kSpecBatch;
    // step 5t (bf16 rows with LDS items): the binade the top-p chain ends in,
    // that of top_p when it is below 1, else [0.5, 1)
    const float tpf = p.top_p;
    const bool skip_on = spec_on && G <= kStage && tpf >= 0x1p-100f && tpf == tpf;
    const int skip_uexp = chain::binade_bits(f2u(tpf < 1.0f ? tpf : 0.75f)).uexp;
    if (!kSorted) {
        for (int i = tid; i < kSpecGroups * kSpecBatches; i += kDThreads) (&sh.spec_cnt[0][0])[i] = 0u;
        if (tid < kSpecBatches) sh.spec_bdone[tid] = 0u;
        if (tid < (kSkipSegs + 31) / 32) sh.skip_flags[tid] = 0u;
        if (tid == 0) {
            sh.skip_built = 0u;
            sh.spec_n = 0u;
            sh.spec_ready = 0u;
            sh.spec_stop = 0u;
        }
    }
    __syncthreads();
    // Top-p cut, draw and near-boundary flag, then the selected value's
    // group. bf16 rows (a few thousand items at most): wave 0 alone, over LDS
    // copies of the items when they fit, else the global arrays. Sorted rows
    // (up to V items): the whole block replays the chains.
    struct Drawn {
        uint32_t pos;
        int item;
        bool near;
    };
    auto draw_wave = [&](const auto& iv) -> Drawn {
        int fl = lane < kDWaves ? sh.ired[lane] : INT_MAX;
        fl = wave_reduce(fl, [](int x, int y) { return min(x, y); });
        // generation.cpp:106-115: min-p stops before element e >= 1 with p_e < minimum.
        uint32_t keff = k;
        if (!any_nan) {
            if (q0 < minimum) keff = 1;
            else if (fl != INT_MAX) keff = min(keff, pre[fl]);
        }
        uint32_t keep, pos;
        int item;
        bool near = false;
        if (any_nan) {
            // NaN probabilities: no cut fires and the walk never stops.
            keep = k;
            pos = k - 1;
            item = wave_find_item(pre, G, pos);
        } else {
            // generation.cpp:105-113: fp32 cumulative, top-p stop needs keep > 0.
            double s2 = static_cast<double>(q0);
            ChainPos cp{0, 1};
            keep = keff;
            constexpr bool kLds = std::is_same_v<std::decay_t<decltype(iv)>, LdsView>;
            const SkipTable sk{kLds && skip_on ? sh.skip_tot : nullptr, sh.skip_flags, &sh.skip_built,
                               kSkipBuilders, skip_uexp};
            if (keff > 1 && wave_chain_f32<false>(iv, G, cp, keff, s2, static_cast<double>(p.top_p), sk))
                keep = cp.elem + 1;
            const float mass = static_cast<float>(s2);
            // random.h:1864-1871 and generation.cpp:118-124.
            const float u = a.uniforms[row];
            const float choice = u * (mass - 0.0f) + 0.0f;
            if (choice > 0.0f && choice < __builtin_inff()) {
                ChainPos w{0, 0};
                double c = static_cast<double>(choice);
                if (wave_chain_f32<true>(iv, G, w, keep, c, 0.0)) {
                    pos = w.elem;
                    item = w.item;
                } else {
                    pos = keep - 1;
                    item = w.item;
                }
            } else if (choice <= 0.0f) {
                pos = 0;
                item = 0;
            } else {  // NaN or +inf: the walk never stops
                pos = keep - 1;
                item = wave_find_item(pre, G, pos);
            }
            // Near-boundary flag: sequential double sums of the probabilities
            // before and through the chosen position, as the oracle defines it.
            double c_before = 0.0;
            if (pos > 0) {
                // exact parallel sum when certified, else the closed-form chain
                double sum = 0.0;
                int mlb = INT_MAX;
                for (int i0 = 0; i0 <= item; i0 += 64) {
                    const int i = i0 + lane;
                    if (i <= item) {
                        const uint32_t st = iv.start(i);
                        const uint32_t en = min(iv.start(i + 1), pos);
                        const float q = iv.addend(i);
                        if (en > st && q > 0.0f) {
                            sum += static_cast<double>(en - st) * static_cast<double>(q);
                            mlb = min(mlb, lsb_exp(q));
                        }
                    }
                }
                sum = wave_reduce(sum, [](double x, double y) { return x + y; });
                mlb = wave_reduce(mlb, [](int x, int y) { return min(x, y); });
                if (sum == 0.0 || mlb >= exp_of(sum) - 51) {
                    c_before = sum;
                } else {
                    ChainPos cp2{0, 1};
                    double sb = static_cast<double>(q0);
                    if (pos > 1) wave_chain<double, false>(iv, G, cp2, pos, sb, __builtin_nan(""));
                    c_before = sb;
                }
            }
            const double c_at = c_before + static_cast<double>(iv.addend(item));
            const double ch = static_cast<double>(choice);
            near = (pos > 0 && __builtin_fabs(ch - c_before) < 1e-6) ||
                   (pos + 1 < keep && __builtin_fabs(ch - c_at) < 1e-6);
        }
        return Drawn{pos, item, near};
    };

    // 6. The selected value's group: items with the same order key are
    //    adjacent; its tokens are the bins with that key (not penalised)
    //    and the penalised tokens with that key. Wave 0.
    auto group = [&](const auto& iv, const Drawn& d) {
        const uint32_t pos = d.pos;
        const int item = d.item;
        const bool near = d.near;
        const float cap = p.softcap;
        auto item_key = [&](int i) { return order_key(u2f(static_cast<uint32_t>(items[i] >> 32))); };
        const uint32_t key = item_key(item);
        int is = item, ie = item;
        for (;;) {  // first item of the group
            const int i = is - 1 - lane;
            const uint64_t m = __ballot(i >= 0 && item_key(i) == key);
            const int run_len = m == ~0ull ? 64 : static_cast<int>(__builtin_ctzll(~m));
            is -= run_len;
            if (run_len < 64) break;
        }
        for (;;) {  // last item of the group
            const int i = ie + 1 + lane;
            const uint64_t m = __ballot(i < G && item_key(i) == key);
            const int run_len = m == ~0ull ? 64 : static_cast<int>(__builtin_ctzll(~m));
            ie += run_len;
            if (run_len < 64) break;
        }
        const uint32_t first = iv.start(is);
        const uint32_t total = iv.start(ie + 1) - first;
        const uint32_t rank = pos - first;
        // Raw keys [blo, bhi] (bf16 bins, or f32 order keys) whose
        // unpenalised final value has this key (empty when blo > bhi).
        uint32_t blo = 1, bhi = 0;
        const bool nan_group = key == kKeyNaN;
        if (!nan_group) {
            if constexpr (kF32) {
                auto fk = [&](uint32_t b) { return order_key(softcap(key_value(b), cap)); };
                // guess: the raw value cap * atanh(v / cap) (v itself without
                // a cap); a raw key's members are usually few
                uint32_t guess = key;
                const float v = key_value(key);
                if (cap > 0.0f && __builtin_fabsf(v) < cap && key != kKeyNaN)
                    guess = order_key(static_cast<float>(static_cast<double>(cap) * atanh(static_cast<double>(v) / cap)));
                blo = wave_partition_point_near(kKeyNegInf, kKeyPosInf + 1, guess, [&](uint32_t b) { return fk(b) < key; });
                bhi = wave_partition_point_near(blo, kKeyPosInf + 1, blo + 32u, [&](uint32_t b) { return fk(b) <= key; }) - 1;
            } else {
                blo = wave_partition_point(kLowBin, kHighBin + 1, [&](uint32_t b) { return bin_key(b, cap) < key; });
                bhi = wave_partition_point(blo, kHighBin + 1, [&](uint32_t b) { return bin_key(b, cap) <= key; }) - 1;
            }
        }
        // penalised tokens with this key: a run of the sorted extras
        uint32_t xs = 0, xe = 0;
        if (E > 0) {
            xs = wave_partition_point(0, E, [&](uint32_t x) { return composite_key(extras[x]) > key; });
            xe = wave_partition_point(xs, E, [&](uint32_t x) { return composite_key(extras[x]) >= key; });
        }
        if (lane == 0) {
            sh.pos = pos;
            sh.item = item;
            sh.near = near ? 1u : 0u;
            sh.group_rank = rank;
            sh.group_total = total;
            sh.blo = blo;
            sh.bhi = bhi;
            sh.nan_group = nan_group ? 1u : 0u;
            sh.gkey = key;
            sh.gx_count = xe - xs;
            sh.forward = (rank <= (total - 1) / 2) ? 1u : 0u;
            sh.token = -1;
        }
        // (the LDS staging area is no longer read, once step 5s has picked;
        // gx_ids reuses it)
        if (!kSorted && spec_on)
            while (__builtin_amdgcn_readfirstlane(
                       __hip_atomic_load(&sh.spec_ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP)) == 0)
                __builtin_amdgcn_s_sleep(2);
        if (!kSorted && skip_on)
            while (__builtin_amdgcn_readfirstlane(__hip_atomic_load(&sh.skip_built, __ATOMIC_ACQUIRE,
                                                                    __HIP_MEMORY_SCOPE_WORKGROUP)) < kSkipBuilders)
                __builtin_amdgcn_s_sleep(2);
        for (uint32_t x = xs + static_cast<uint32_t>(lane); x < xe; x += 64)
            sh.gx_ids[x - xs] = composite_index(extras[x]);
    };

    // 5s. bf16 rows: while wave 0 draws, the other waves count, per batch of
    //     the token scan below, the tokens of the groups the draw is likely
    //     to select. Wave 1 finds the item where the exact cumulative
    //     probability crosses u * min(top_p, mass through the cuts) (the f32
    //     chains end within a small fraction of an item of it), takes the
    //     groups of the items around it, and from the element there predicts
    //     the scan's direction and how many batches it passes before the
    //     token (with a margin). The counting waves then count each group's
    //     unpenalised tokens in those batches, from the scan's end inward, as
    //     the scan's match would. The scan skips the counted batches before
    //     the token's by those counts (plus the group's penalised ids there),
    //     so it finds the token it would find anyway; a group not among the
    //     candidates, or batches the count did not finish before wave 0 did,
    //     are scanned as before. group() waits for the pick before it
    //     reuses the LDS copies of the items.
    auto spec_pick = [&](const auto& iv) {  // wave 1
        int fl = lane < kDWaves ? sh.ired[lane] : INT_MAX;
        fl = wave_reduce(fl, [](int x, int y) { return min(x, y); });
        uint32_t keff = k;
        if (q0 < minimum) keff = 1;
        else if (fl != INT_MAX) keff = min(keff, pre[fl]);
        const double u = static_cast<double>(a.uniforms[row]);
        const double tp = static_cast<double>(p.top_p);
        auto mass = [&](int i) -> double {  // i < G
            const uint32_t st = min(iv.start(i), keff), en = min(iv.start(i + 1), keff);
            return static_cast<double>(en - st) * static_cast<double>(iv.addend(i));
        };
        // the items in 64 runs, one per lane; then the crossing run, 64 at a time
        const int B = (G + 63) / 64;
        const int ib = min(lane * B, G), ie = min(ib + B, G);
        double part = 0.0;
        for (int i0 = ib; i0 < ie; i0 += 8) {
            double m[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) m[j] = mass(min(i0 + j, ie - 1));  // clamped: no conditional load
#pragma unroll
            for (int j = 0; j < 8; ++j) part += i0 + j < ie ? m[j] : 0.0;
        }
        const double incl = wave::incl_f64(part);
        const double total = wave::readlane_f64(incl, 63);
        const double c = u * (total >= tp ? tp : total);
        const uint64_t bl = __ballot(ib < ie && incl >= c);
        int ic = -1;
        double before = 0.0;
        if (bl) {
            const int L = static_cast<int>(__builtin_ctzll(bl));
            double base = wave::readlane_f64(incl - part, L);
            const int lb = L * B, le = min(lb + B, G);
            for (int i0 = lb; i0 < le; i0 += 64) {
                const int i = i0 + lane;
                const double mi = i < le ? mass(i) : 0.0;
                const double inc = base + wave::incl_f64(mi);
                const uint64_t b = __ballot(i < le && inc >= c);
                if (b) {
                    const int f = static_cast<int>(__builtin_ctzll(b));
                    ic = i0 + f;
                    before = wave::readlane_f64(inc - mi, f);
                    break;
                }
                base = wave::readlane_f64(inc, 63);
            }
            if (ic < 0) ic = le - 1;
        }
        uint32_t n = 0, ulo = kHighBin + 1, uhi = 0, fwd = 1, nbat = 0;
        if (ic >= 0) {
            const float cap = p.softcap;
            auto item_key = [&](int i) { return order_key(u2f(static_cast<uint32_t>(items[i] >> 32))); };
            // distinct keys of items ic - kSpecBefore .. ic + kSpecAfter, descending
            const int ij = ic - kSpecBefore + lane;
            const bool in = lane <= kSpecBefore + kSpecAfter && ij >= 0 && ij < G;
            const uint32_t kj = in ? item_key(min(max(ij, 0), G - 1)) : 0u;
            const uint32_t kp = __shfl_up(kj, 1);
            const bool take = in && kj != kKeyNaN && !(lane > 0 && ij > 0 && kp == kj);
            const uint64_t tm = __ballot(take);
            n = static_cast<uint32_t>(__popcll(tm));
            if (n > 0) {
                const uint32_t khi = wave::readlane(kj, static_cast<int>(__builtin_ctzll(tm)));
                const uint32_t klo = wave::readlane(kj, 63 - static_cast<int>(__builtin_clzll(tm)));
                // the bins of keys [klo, khi]: [r0, r1)
                const uint32_t r0 =
                    wave_partition_point(kLowBin, kHighBin + 1, [&](uint32_t b) { return bin_key(b, cap) < klo; });
                const uint32_t r1 =
                    wave_partition_point(r0, kHighBin + 1, [&](uint32_t b) { return bin_key(b, cap) <= khi; });
                const bool narrow = r1 - r0 <= 64;
                const uint32_t bk = narrow && r0 + lane < r1 ? bin_key(r0 + lane, cap) : 0xFFFFFFFFu;
                uint64_t rest = tm;
                for (uint32_t c = 0; c < n; ++c) {
                    const int l = static_cast<int>(__builtin_ctzll(rest));
                    rest &= rest - 1;
                    const uint32_t key = wave::readlane(kj, l);
                    uint32_t blo, bhi;
                    if (narrow) {  // bin_key is monotone: count the bins below / through key
                        blo = r0 + static_cast<uint32_t>(__popcll(__ballot(r0 + lane < r1 && bk < key)));
                        bhi = r0 + static_cast<uint32_t>(__popcll(__ballot(r0 + lane < r1 && bk <= key))) - 1;
                    } else {
                        blo = wave_partition_point(r0, r1, [&](uint32_t b) { return bin_key(b, cap) < key; });
                        bhi = wave_partition_point(blo, r1, [&](uint32_t b) { return bin_key(b, cap) <= key; }) - 1;
                    }
                    if (lane == 0) {
                        sh.spec_key[c] = key;
                        sh.spec_blo[c] = blo;
                        sh.spec_bhi[c] = bhi;
                    }
                    if (blo <= bhi) {
                        ulo = min(ulo, blo);
                        uhi = max(uhi, bhi);
                    }
                }
            }
            // The predicted element, its rank in its group (the items of
            // one key, within a few items of ic), and the batches the scan
            // would pass before reaching it: the members are spread over the
            // row, so the want-th from the scan's end lies near V * (want + 1)
            // / (total + 1). Margins: the chains' drift (about 1.5e-4 of
            // probability, in elements of this item) and three binomial
            // standard deviations, plus one batch. When the drift leaves the
            // direction open, every batch.
            const uint32_t key = item_key(ic);
            const uint64_t mb = __ballot(ic - 1 - lane >= 0 && item_key(max(ic - 1 - lane, 0)) == key);
            const uint64_t ma = __ballot(ic + 1 + lane < G && item_key(min(ic + 1 + lane, G - 1)) == key);
            const int is = ic - (mb == ~0ull ? 64 : static_cast<int>(__builtin_ctzll(~mb)));
            const int ie2 = ic + (ma == ~0ull ? 64 : static_cast<int>(__builtin_ctzll(~ma)));
            const double q = static_cast<double>(aux[ic]);
            const uint32_t cnt_ic = pre[ic + 1] - pre[ic];
            double off = q > 0.0 ? (c - before) / q : 0.0;
            off = off < 0.0 ? 0.0 : off;
            const uint32_t within = off >= static_cast<double>(cnt_ic) ? cnt_ic - 1 : static_cast<uint32_t>(off);
            const uint32_t first = pre[is], tot = pre[ie2 + 1] - first;
            const uint32_t rank = pre[ic] + within - first;
            fwd = rank <= (tot - 1) / 2 ? 1u : 0u;
            const uint32_t want = fwd ? rank : tot - 1 - rank;
            const double drift = q > 0.0 ? 1.5e-4 / q : static_cast<double>(tot);
            const double mid = (static_cast<double>(tot) - 1.0) * 0.5;
            const bool sure = static_cast<double>(rank) + drift <= mid || static_cast<double>(rank) - drift > mid;
            const double pf = (static_cast<double>(want) + 1.0 + drift) / (static_cast<double>(tot) + 1.0);
            const double pc = pf < 1.0 ? pf : 1.0;
            const double hi = pc + 3.0 * __builtin_sqrt(pc * (1.0 - pc) / (static_cast<double>(tot) + 1.0));
            const int nb = (V + kSpecBatch - 1) / kSpecBatch;
            const double bats = hi * static_cast<double>(V) / kSpecBatch + 1.0;
            // a direction the drift leaves open: every batch, for either end
            nbat = !sure || bats >= static_cast<double>(nb) ? static_cast<uint32_t>(nb) : static_cast<uint32_t>(bats);
        }
        if (lane == 0) {
            sh.spec_ulo = ulo;
            sh.spec_uhi = uhi;
            sh.spec_n = n;
            sh.spec_fwd = fwd;
            sh.spec_nbat = nbat;
            __hip_atomic_store(&sh.spec_ready, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    };
    // 5t. bf16 rows with LDS items: waves 2-7 build the top-p chain's skip
    //     table (chain_wave.h SkipTable) for the binade it ends in, where it
    //     spends most of its steps (C4: items 711-2830 of about 3050), before
    //     they count. The chain passes a segment by its total only when that
    //     is exactly what the segment's step would add.
    auto skip_build = [&]() {
        int fl = lane < kDWaves ? sh.ired[lane] : INT_MAX;
        fl = wave_reduce(fl, [](int x, int y) { return min(x, y); });
        uint32_t keff = k;  // as the draw's (generation.cpp:106-115)
        if (q0 < minimum) keff = 1;
        else if (fl != INT_MAX) keff = min(keff, pre[fl]);
        const int nseg = (G + kSkipSeg - 1) / kSkipSeg;
        for (int sg = wave - 2; sg < nseg; sg += kSkipBuilders) {
            uint32_t lt = 0;
            bool ev = false;
#pragma unroll
            for (int j = 0; j < LdsView::kPerLane; ++j) {
                const int i = sg * kSkipSeg + lane * LdsView::kPerLane + j;
                if (i < G) {
                    const uint32_t n = min(sh.st.pre[i + 1], keff) - min(sh.st.pre[i], keff);
                    uint32_t D;
                    bool tie, big;
                    chain::step_bits(f2u(sh.st.add[i]), skip_uexp, D, tie, big);
                    if (n) {
                        ev = ev || tie || big;
                        const uint64_t t = static_cast<uint64_t>(n) * D;
                        lt += t > 0x1000000u ? 0x1000000u : static_cast<uint32_t>(t);
                    }
                }
            }
            lt = min(lt, 0x1000000u);
            const uint32_t tot = wave::readlane(wave::incl_add(lt), 63);  // <= 64 * 2^24
            const bool any = __ballot(ev) != 0ull;
            if (lane == 0) {
                sh.skip_tot[sg] = min(tot, 0x1000000u);
                if (any) atomicOr(&sh.skip_flags[sg >> 5], 1u << (sg & 31));
            }
        }
        if (lane == 0) __hip_atomic_fetch_add(&sh.skip_built, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    };
    auto spec_count = [&]() {  // the counting waves
        while (__builtin_amdgcn_readfirstlane(
                   __hip_atomic_load(&sh.spec_ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP)) == 0)
            __builtin_amdgcn_s_sleep(2);
        const uint32_t n = sh.spec_n;
        const uint32_t ulo = sh.spec_ulo, uhi = sh.spec_uhi;
        const bool fwd = sh.spec_fwd != 0;
        const int nb = (V + kSpecBatch - 1) / kSpecBatch;
        constexpr int kPerBatch = kSpecBatch / kSpecBlock;
        const int nblk = static_cast<int>(sh.spec_nbat) * kPerBatch;  // blocks counted, from the scan's end
        if (n == 0) return;
        const uint32_t span = uhi - ulo;  // (no bin passes when every range is empty: ulo > uhi)
        uint32_t cb[kSpecGroups], ch[kSpecGroups];
#pragma unroll
        for (int c = 0; c < kSpecGroups; ++c) {
            cb[c] = c < static_cast<int>(n) ? sh.spec_blo[c] : 1u;
            ch[c] = c < static_cast<int>(n) ? sh.spec_bhi[c] : 0u;
        }
        const uint16_t* rowp = static_cast<const uint16_t*>(a.logits) + static_cast<int64_t>(row) * a.row_stride;
        const bool vec = a.vec_ok != 0;
        auto block_of = [&](int j) { return fwd ? j : nb * kPerBatch - 1 - j; };
        auto load32 = [&](int j, uint32_t* w, uint32_t& valid) {
            const int lo = block_of(j) * kSpecBlock + lane * 32;
            valid = 0;
            if (vec && lo + 32 <= V) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint4 v = *reinterpret_cast<const uint4*>(rowp + lo + q * 8);
                    w[4 * q + 0] = v.x; w[4 * q + 1] = v.y; w[4 * q + 2] = v.z; w[4 * q + 3] = v.w;
                }
                valid = 0xFFFFFFFFu;
            } else {
                for (int h = 0; h < 16; ++h) w[h] = 0;
                for (int h = 0; h < 32; ++h) {
                    if (lo + h < V) {
                        w[h >> 1] |= static_cast<uint32_t>(rowp[lo + h]) << ((h & 1) * 16);
                        valid |= 1u << h;
                    }
                }
            }
        };
        const int slot = __builtin_popcount(kSpecWaves & ((1u << wave) - 1u));
        uint32_t cur[16], nxt[16];
        uint32_t cval = 0, nval = 0;
        if (slot < nblk) load32(slot, cur, cval);
        for (int j = slot; j < nblk; j += kSpecCounters) {
            if (__builtin_amdgcn_readfirstlane(
                    __hip_atomic_load(&sh.spec_stop, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) != 0)
                break;
            const int blk = block_of(j);
            const int lo = blk * kSpecBlock + lane * 32;
            if (j + kSpecCounters < nblk) load32(j + kSpecCounters, nxt, nval);
            uint32_t hits = 0;
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                if (bin_of(cur[q] & 0xFFFFu) - ulo <= span) hits |= 1u << (2 * q);
                if (bin_of(cur[q] >> 16) - ulo <= span) hits |= 2u << (2 * q);
            }
            hits &= cval;
            if (pen && hits) hits &= ~bitmap[lo >> 5];  // 32 tokens at a multiple of 32: one word
            const int batch = blk / kPerBatch;
            while (hits) {
                const int h = __builtin_ctz(hits);
                hits &= hits - 1u;
                uint32_t wv = 0;
#pragma unroll
                for (int q = 0; q < 16; ++q) wv = (h >> 1) == q ? cur[q] : wv;
                const uint32_t bin = bin_of((h & 1) ? wv >> 16 : wv & 0xFFFFu);
                int c = -1;
#pragma unroll
                for (int cc = 0; cc < kSpecGroups; ++cc)
                    if (bin >= cb[cc] && bin <= ch[cc]) c = cc;
                if (c >= 0) atomicAdd(&sh.spec_cnt[c][batch], 1u);
            }
            if (lane == 0) atomicAdd(&sh.spec_bdone[batch], 1u);  // after this block's counts (LDS order)
#pragma unroll
            for (int q = 0; q < 16; ++q) cur[q] = nxt[q];
            cval = nval;
        }
    };
    if constexpr (kSorted) {
        // Every value below is uniform across the block (block_chain's
        // results are), as block_chain requires of its arguments.
        int fl = INT_MAX;
        for (int w = 0; w < kDWaves; ++w) fl = min(fl, sh.ired[w]);
        // generation.cpp:106-115: min-p stops before element e >= 1 with p_e < minimum.
        uint32_t keff = k;
        if (!any_nan) {
            if (q0 < minimum) keff = 1;
            else if (fl != INT_MAX) keff = min(keff, pre[fl]);
        }
        Drawn d{0, 0, false};
        if (any_nan) {
            // NaN probabilities: no cut fires and the walk never stops.
            d.pos = k - 1;
            d.item = wave_find_item(pre, G, d.pos);
        } else {
            // generation.cpp:105-113: fp32 cumulative, top-p stop needs keep > 0.
            double s2 = static_cast<double>(q0);
            ChainPos cp{0, 1};
            uint32_t keep = keff;
            if (keff > 1 && bchain::block_chain<bchain::F32Acc, false, kDThreads>(pre, aux, inv, G, cp, keff, s2,
                                                                                   static_cast<double>(p.top_p), sh.bc))
                keep = cp.elem + 1;
            const float mass = static_cast<float>(s2);
            // random.h:1864-1871 and generation.cpp:118-124.
            const float u = a.uniforms[row];
            const float choice = u * (mass - 0.0f) + 0.0f;
            if (choice > 0.0f && choice < __builtin_inff()) {
                ChainPos w{0, 0};
                double c = static_cast<double>(choice);
                const bool stop =
                    bchain::block_chain<bchain::F32Acc, true, kDThreads>(pre, aux, inv, G, w, keep, c, 0.0, sh.bc);
                d.pos = stop ? w.elem : keep - 1;
                d.item = w.item;
            } else if (choice <= 0.0f) {
                d.pos = 0;
                d.item = 0;
            } else {  // NaN or +inf: the walk never stops
                d.pos = keep - 1;
                d.item = wave_find_item(pre, G, d.pos);
            }
            // Near-boundary flag: sequential double sums of the probabilities
            // before and through the chosen position, as the oracle defines
            // it: an exact parallel sum when certified, else the replay.
            double c_before = 0.0;
            if (d.pos > 0) {
                double sum = 0.0;
                int mlb = INT_MAX;
                constexpr int kU = 16;
                for (int base = 0; base <= d.item; base += kDThreads * kU) {
                    uint32_t stv[kU], env[kU];
                    float qv[kU];
#pragma unroll
                    for (int u2 = 0; u2 < kU; ++u2) {  // clamped to d.item: no conditional load
                        const int i = min(base + u2 * kDThreads + tid, d.item);
                        stv[u2] = pre[i];
                        env[u2] = pre[i + 1];
                        qv[u2] = aux[i] * inv;
                    }
#pragma unroll
                    for (int u2 = 0; u2 < kU; ++u2) {
                        const bool in = base + u2 * kDThreads + tid <= d.item;
                        const uint32_t en = min(env[u2], d.pos);
                        if (in && en > stv[u2] && qv[u2] > 0.0f) {
                            sum += static_cast<double>(en - stv[u2]) * static_cast<double>(qv[u2]);
                            mlb = min(mlb, lsb_exp(qv[u2]));
                        }
                    }
                }
                sum = wave_reduce(sum, [](double x, double y) { return x + y; });
                mlb = wave_reduce(mlb, [](int x, int y) { return min(x, y); });
                __syncthreads();  // every earlier reader of dred / ired is done
                if (lane == 0) {
                    sh.dred[wave] = sum;
                    sh.ired[wave] = mlb;
                }
                __syncthreads();
                sum = 0.0;
                mlb = INT_MAX;
                for (int w = 0; w < kDWaves; ++w) {
                    sum += sh.dred[w];
                    mlb = min(mlb, sh.ired[w]);
                }
                if (sum == 0.0 || mlb >= exp_of(sum) - 51) {
                    c_before = sum;
                } else {
                    ChainPos cp2{0, 1};
                    double sb = static_cast<double>(q0);
                    if (d.pos > 1)
                        bchain::block_chain<bchain::F64Acc, false, kDThreads>(pre, aux, inv, G, cp2, d.pos, sb,
                                                                              __builtin_nan(""), sh.bc);
                    c_before = sb;
                }
            }
            const double c_at = c_before + static_cast<double>(aux[d.item] * inv);
            const double ch = static_cast<double>(choice);
            d.near = (d.pos > 0 && __builtin_fabs(ch - c_before) < 1e-6) ||
                     (d.pos + 1 < keep && __builtin_fabs(ch - c_at) < 1e-6);
        }
        if (wave == 0) group(GlobalView{pre, aux}, d);
    } else if (wave == 0) {
        // the draw's serial chains first, when the counting waves share its SIMD
        if (spec_on) __builtin_amdgcn_s_setprio(3);
        if (G <= kStage) {
            const LdsView v{sh.st.pre, sh.st.add};
            group(v, draw_wave(v));
        } else {
            const GlobalView v{pre, aux};
            group(v, draw_wave(v));
        }
        if (spec_on) __builtin_amdgcn_s_setprio(0);
        if (spec_on && lane == 0) __hip_atomic_store(&sh.spec_stop, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    } else if (spec_on && ((kSpecWaves >> wave) & 1u)) {
        if (wave == 1) {
            if (G <= kStage) spec_pick(LdsView{sh.st.pre, sh.st.add});
            else spec_pick(GlobalView{pre, aux});
        }
        if (skip_on && wave >= 2) skip_build();
        spec_count();
    }
    __syncthreads();

    // Locate the token: the rank-th lowest index of the group (or the
    // (total-1-rank)-th highest), in batches of 16384 tokens from that end;
    // the next batch's loads are in flight while this one is scanned. Each
    // wave reads 2048 consecutive tokens of a batch in 16-byte chunks, lane l
    // taking chunk l of each row of 64 chunks, so that every load reads 1 KB
    // of consecutive bytes (a lane's own tokens are kChunks chunks, one per
    // row). Scan order inside a batch is thus wave, chunk row, lane, token.
    // A token is in the group when its raw key is in [blo, bhi] and it is
    // not penalised; penalised tokens of the group are the extras run (bf16)
    // or are evaluated where the bitmap marks them (f32).
    {
        constexpr int kPer = 32;                                      // tokens per thread per batch
        constexpr int kBatch = kDThreads * kPer;
        constexpr int kW = kPer * static_cast<int>(sizeof(T)) / 4;    // 32-bit words per thread per batch
        constexpr int kTokC = 16 / static_cast<int>(sizeof(T));      // tokens per 16-byte chunk
        constexpr int kChunks = kPer / kTokC;                         // chunks per thread per batch
        constexpr int kRowC = 64 * kTokC;                             // tokens per chunk row of a wave
        constexpr int kWaveSpan = 64 * kPer;                          // tokens per wave per batch
        static_assert(kWaveSpan == 64 * 32, "one history bitmap word per lane covers a wave's tokens");
        const bool fwd = sh.forward != 0;
        uint32_t want = fwd ? sh.group_rank : sh.group_total - 1 - sh.group_rank;
        const uint32_t blo = sh.blo, bhi = sh.bhi;
        const bool nan_group = sh.nan_group != 0;
        const uint32_t gkey = sh.gkey;
        const uint32_t gx = sh.gx_count;
        const T* rowp = static_cast<const T*>(a.logits) + static_cast<int64_t>(row) * a.row_stride;
        const bool vec = a.vec_ok != 0;
        const float cap = p.softcap;
        const float rpen = p.repetition_penalty;
        // penalised ids of the group in [lo, hi) (bf16 extras)
        auto gx_in = [&](uint32_t lo, uint32_t hi) -> uint32_t {
            if (gx == 0) return 0;
            uint32_t a0 = 0, a1 = gx;
            while (a0 < a1) { const uint32_t m = (a0 + a1) >> 1; if (sh.gx_ids[m] < lo) a0 = m + 1; else a1 = m; }
            uint32_t b0 = a0, b1 = gx;
            while (b0 < b1) { const uint32_t m = (b0 + b1) >> 1; if (sh.gx_ids[m] < hi) b0 = m + 1; else b1 = m; }
            return b0 - a0;
        };
        // First token of this thread's chunk q of the batch at token B.
        auto chunk_tok = [&](int B, int q) { return B + wave * kWaveSpan + q * kRowC + lane * kTokC; };
        // Any batch: its words, the valid tokens, and the history bitmap's
        // word B / 32 + wave * 64 + lane (the wave's tokens of the batch lie
        // in its 64 words).
        auto load_any = [&](int B, uint32_t* w, uint32_t& valid, uint32_t& bw) {
            bw = pen ? bitmap[min((B >> 5) + wave * 64 + lane, (V - 1) >> 5)] : 0u;  // clamped: no conditional load
            valid = 0;
            if (vec && chunk_tok(B, kChunks - 1) + kTokC <= V) {
                const T* p0 = rowp + chunk_tok(B, 0);
#pragma unroll
                for (int q = 0; q < kChunks; ++q) {
                    const uint4 v = *reinterpret_cast<const uint4*>(p0 + q * kRowC);
                    w[4 * q + 0] = v.x; w[4 * q + 1] = v.y; w[4 * q + 2] = v.z; w[4 * q + 3] = v.w;
                }
                valid = 0xFFFFFFFFu;
            } else {
                for (int h = 0; h < kW; ++h) w[h] = 0;
                for (int q = 0; q < kChunks; ++q) {
                    for (int j = 0; j < kTokC; ++j) {
                        const int t = chunk_tok(B, q) + j;
                        const int h = q * kTokC + j;
                        if (t < V) {
                            if constexpr (sizeof(T) == 4) w[h] = f2u(rowp[t]);
                            else w[h >> 1] |= static_cast<uint32_t>(rowp[t]) << ((h & 1) * 16);
                            valid |= 1u << h;
                        }
                    }
                }
            }
        };
        // A batch wholly inside a 16-byte aligned row: a fixed set of loads
        // with no branch around them. The bitmap is all zero when no history
        // applies: its first word serves.
        auto load_full = [&](int B, uint32_t* w, uint32_t& valid, uint32_t& bw) {
            bw = bitmap[pen ? (B >> 5) + wave * 64 + lane : 0];
            const T* p0 = rowp + chunk_tok(B, 0);
#pragma unroll
            for (int q = 0; q < kChunks; ++q) {
                const uint4 v = *reinterpret_cast<const uint4*>(p0 + q * kRowC);
                w[4 * q + 0] = v.x; w[4 * q + 1] = v.y; w[4 * q + 2] = v.z; w[4 * q + 3] = v.w;
            }
            valid = 0xFFFFFFFFu;
        };
        // The penalised ones among the thread's tokens: chunk q of lane l
        // lies in the bitmap word that lane (q * kRowC + l * kTokC) / 32 loaded.
        auto pen_mask = [&](int B, uint32_t bw, uint32_t valid) -> uint32_t {
            if (!pen) return 0u;
            uint32_t pm = 0;
#pragma unroll
            for (int q = 0; q < kChunks; ++q) {
                const uint32_t word = static_cast<uint32_t>(__shfl(static_cast<int>(bw), (q * kRowC + lane * kTokC) >> 5, 64));
                const uint32_t at = static_cast<uint32_t>(chunk_tok(B, q)) & 31u;
                pm |= ((word >> at) & ((1u << kTokC) - 1u)) << (q * kTokC);
            }
            return pm & valid;
        };
        // Group members among the thread's tokens (bf16: not counting the
        // penalised ones, which the extras run supplies). f32: branch-free
        // per token, one range test (raw key - blo <= bhi - blo) and a bit.
        auto match = [&](int B, const uint32_t* w, uint32_t valid, uint32_t bw) -> uint32_t {
            const uint32_t pw = pen_mask(B, bw, valid);
            if constexpr (kF32) {
                const uint32_t span = bhi - blo;
                const uint32_t some = blo <= bhi ? 0xFFFFFFFFu : 0u;  // (empty when blo > bhi)
                uint32_t in = 0;
                auto value = [&](int h) {
                    return sizeof(T) == 4 ? u2f(w[h]) : u2f(((w[h >> 1] >> ((h & 1) * 16)) & 0xFFFFu) << 16);
                };
                if (nan_group) {
#pragma unroll
                    for (int h = 0; h < kPer; ++h) {
                        const float x = value(h);
                        in |= (x != x ? 1u : 0u) << h;
                    }
                    return in & valid;
                }
                if (blo > 0x80000000u || bhi < 0x80000000u) {
                    // keys of one sign: the raw bits of that sign's floats
                    // follow the keys (positive: key = bits | 2^31; negative:
                    // key = ~bits), and the others, zero and NaN fall outside
                    const uint32_t rlo = blo > 0x80000000u ? (blo & 0x7FFFFFFFu) : ~bhi;
#pragma unroll
                    for (int h = 0; h < kPer; ++h) in |= (f2u(value(h)) - rlo <= span ? 1u : 0u) << h;
                } else {
#pragma unroll
                    for (int h = 0; h < kPer; ++h) in |= (order_key(value(h)) - blo <= span ? 1u : 0u) << h;
                }
                uint32_t mm = in & some & valid & ~pw;
                for (uint32_t b = pw; b; b &= b - 1u) {
                    const int h = __builtin_ctz(b);
                    // the token's value from the loaded words (a select
                    // chain: a per-lane index into registers)
                    uint32_t wv = 0;
#pragma unroll
                    for (int q = 0; q < kW; ++q) wv = (sizeof(T) == 4 ? h : h >> 1) == q ? w[q] : wv;
                    const float x = sizeof(T) == 4 ? u2f(wv) : u2f(((wv >> ((h & 1) * 16)) & 0xFFFFu) << 16);
                    const float f = penalize(softcap(x, cap), rpen);
                    if (order_key(f) == gkey) mm |= 1u << h;
                }
                return mm;
            } else {
                // (bf16 rows run two workgroups per CU: this form keeps the
                // kernel within 128 VGPRs)
                auto bin_match = [&](uint32_t bits16) {
                    const uint32_t bin = bin_of(bits16);
                    return nan_group ? bin_is_nan(bin) : (bin >= blo && bin <= bhi);
                };
                uint32_t mm = 0;
#pragma unroll
                for (int h = 0; h < kPer; ++h) {
                    if (((valid >> h) & 1u) && bin_match((w[h >> 1] >> ((h & 1) * 16)) & 0xFFFFu)) mm |= 1u << h;
                }
                return mm & ~pw;
            }
        };
        // bf16: the group's penalised ids in chunk q of the thread (the
        // extras run).
        auto gx_chunk = [&](int B, int q) -> uint32_t {
            const int t0 = chunk_tok(B, q);
            return (gx && t0 < V) ? gx_in(static_cast<uint32_t>(t0), static_cast<uint32_t>(min(t0 + kTokC, V))) : 0u;
        };
        const int nb = (V + kBatch - 1) / kBatch;
        // Batches the speculative counts (step 5s) show to hold fewer than
        // `want` more tokens of the group are skipped.
        int bi0 = 0;
        if constexpr (!kF32) {
            static_assert(kF32 || kBatch == kSpecBatch, "the counts are per token-scan batch");
            if (spec_on && !nan_group) {
                int c = -1;
                for (uint32_t cc = 0; cc < sh.spec_n; ++cc)
                    if (sh.spec_key[cc] == gkey) c = static_cast<int>(cc);
                if (c >= 0) {
                    while (bi0 + 1 < nb) {
                        const int batch = fwd ? bi0 : nb - 1 - bi0;
                        if (sh.spec_bdone[batch] != static_cast<uint32_t>(kSpecBatch / kSpecBlock)) break;
                        const uint32_t b0 = static_cast<uint32_t>(batch * kBatch);
                        const uint32_t b1 = static_cast<uint32_t>(min((batch + 1) * kBatch, V));
                        const uint32_t cnt = sh.spec_cnt[c][batch] + gx_in(b0, b1);
                        if (want < cnt) break;
                        want -= cnt;
                        ++bi0;
                    }
                }
            }
        }
        auto batch_base = [&](int bi) { return (fwd ? bi : nb - 1 - bi) * kBatch; };
        // One batch; true when it holds the token (the scan ends there). The
        // batch's count is a block sum (the waves' sums through LDS, two
        // buffers in turn: consecutive batches are one barrier apart); only
        // the batch that holds the token orders its members.
        auto scan_batch = [&](int bi, const uint32_t* w, uint32_t valid, uint32_t bw) -> bool {
            const int B = batch_base(bi);
            const uint32_t mm = match(B, w, valid, bw);
            uint32_t cnt = static_cast<uint32_t>(__popc(mm));
            if constexpr (!kF32) {
                if (gx) {
                    for (int q = 0; q < kChunks; ++q) cnt += gx_chunk(B, q);
                }
            }
            uint32_t* wt = sh.tscan[bi & 1];
            const uint32_t wsum = wave::readlane(wave_incl_u32(cnt), 63);
            if (lane == 0) wt[wave] = wsum;
            __syncthreads();
            uint32_t tot = 0;
#pragma unroll
            for (int w2 = 0; w2 < kDWaves; ++w2) tot += wt[w2];
            if (want >= tot) {
                want -= tot;
                return false;
            }
            // The token's wave, then its chunk row, lane and token, in scan order.
            uint32_t r = want;
            int tw = -1;
#pragma unroll
            for (int s2 = 0; s2 < kDWaves; ++s2) {
                const int w2 = fwd ? s2 : kDWaves - 1 - s2;
                if (tw < 0) {
                    if (r < wt[w2]) tw = w2;
                    else r -= wt[w2];
                }
            }
            if (wave == tw) {
                for (int s2 = 0; s2 < kChunks; ++s2) {
                    const int q = fwd ? s2 : kChunks - 1 - s2;
                    uint32_t cq = static_cast<uint32_t>(__popc((mm >> (q * kTokC)) & ((1u << kTokC) - 1u)));
                    if constexpr (!kF32) cq += gx_chunk(B, q);
                    const uint32_t incl = wave_incl_u32(cq);
                    const uint32_t rowtot = wave::readlane(incl, 63);
                    if (r >= rowtot) {
                        r -= rowtot;
                        continue;
                    }
                    const uint32_t ex = fwd ? incl - cq : rowtot - incl;
                    if (r >= ex && r < ex + cq) {
                        uint32_t r2 = r - ex;
                        int found = -1;
                        const int t0 = chunk_tok(B, q);
                        for (int s3 = 0; s3 < kTokC && found < 0; ++s3) {
                            const int j = fwd ? s3 : kTokC - 1 - s3;
                            const int h = q * kTokC + j;
                            if (!((valid >> h) & 1u)) continue;
                            const uint32_t idx = static_cast<uint32_t>(t0 + j);
                            uint32_t here = (mm >> h) & 1u;
                            if constexpr (!kF32) {
                                if (!here && gx) here = gx_in(idx, idx + 1);
                            }
                            if (here) {
                                if (r2 == 0) found = static_cast<int>(idx);
                                else --r2;
                            }
                        }
                        sh.token = found;
                    }
                    break;
                }
            }
            return true;
        };
        // Scan indices [b0, b1) with two buffers in turn, the next batch's
        // loads in flight while this one is matched and scanned, and no
        // register copy between batches. The next loads are issued on every
        // turn (the last batch again when none is left): with a load issued
        // on one path only, the compiler's wait before the match covers
        // every load in flight, the next batch's included.
        auto pipelined = [&](auto&& loader, int b0, int b1) -> bool {
            if (b0 >= b1) return false;
            uint32_t wa[kW], wb[kW];
            uint32_t va = 0, vb = 0, bwa = 0, bwb = 0;
            loader(batch_base(b0), wa, va, bwa);
            for (int bi = b0; bi < b1; bi += 2) {
                // (distinct markers keep the compiler from folding the two
                // halves into one loop body over a single buffer)
                asm volatile("; token scan: buffer b in flight");
                loader(batch_base(min(bi + 1, b1 - 1)), wb, vb, bwb);
                if (scan_batch(bi, wa, va, bwa)) return true;
                if (bi + 1 >= b1) break;
                asm volatile("; token scan: buffer a in flight");
                loader(batch_base(min(bi + 2, b1 - 1)), wa, va, bwa);
                if (scan_batch(bi + 1, wb, vb, bwb)) return true;
            }
            return false;
        };
        if (vec) {
            // the last batch (scan index nb - 1 forward, 0 backward) may be
            // partial: it takes the general loads, the full ones the fixed set
            const bool partial = V % kBatch != 0;
            int b0 = bi0, b1 = nb;
            bool done = false;
            if (partial && !fwd && b0 == 0) {
                uint32_t w[kW], v = 0, bw = 0;
                load_any(batch_base(0), w, v, bw);
                done = scan_batch(0, w, v, bw);
                b0 = 1;
            }
            if (partial && fwd) b1 = nb - 1;
            if (!done) done = pipelined(load_full, b0, b1);
            if (!done && partial && fwd && bi0 <= nb - 1) {
                uint32_t w[kW], v = 0, bw = 0;
                load_any(batch_base(nb - 1), w, v, bw);
                (void)scan_batch(nb - 1, w, v, bw);
            }
        } else {
            (void)pipelined(load_any, bi0, nb);
        }
    }
    __syncthreads();
    finish(sh.token, kSorted ? aux[sh.item] * inv : aux[sh.item], sh.near ? GE_FLAG_NEAR_BOUNDARY : 0);
}

// The per-row pointers of rows [r0, r0 + n) of a call, as a call of its own
// that uses workspace rows [0, n).
DevArgs slice_rows(const DevArgs& a, int r0, int n) {
    DevArgs s = a;
    const size_t esize = a.dtype == GE_DTYPE_BF16 ? 2 : 4;
    s.logits = static_cast<const char*>(a.logits) + esize * static_cast<size_t>(a.row_stride) * static_cast<size_t>(r0);
    s.rows = n;
    if (a.row_params) s.row_params = a.row_params + r0;
    if (a.history_offsets) s.history_offsets = a.history_offsets + r0;
    if (a.ring) s.ring = a.ring + static_cast<int64_t>(r0) * a.ring_capacity;
    if (a.ring_len) s.ring_len = a.ring_len + r0;
    if (a.uniforms) s.uniforms = a.uniforms + r0;
    s.tokens = a.tokens + r0;
    if (a.probs) s.probs = a.probs + r0;
    if (a.flags) s.flags = a.flags + r0;
    if (a.done) s.done = a.done + r0;
    s.fo_row0 = a.fo_row0 + r0;
    return s;
}

}  // namespace

namespace {

// Rows [0, a.rows) through the sort-based kernels, as many per launch pair as
// the workspace holds at the f32 stride (at least one, by construction).
// The items of f32 rows [0, s.rows) through the many-workgroup sort: tiles
// of 4096 keys, one workgroup each, one kernel per step.
hipError_t split_sort_f32(const DevArgs& s, hipStream_t stream) {
    const int T = fo_split_tiles(s.vocab);
    const dim3 tiles(static_cast<unsigned>(T), static_cast<unsigned>(s.rows));
    const dim3 rows(static_cast<unsigned>(s.rows));
    // A few rows: each keys tile builds its own bitmap words, and each
    // scatter tile scans its row's counts itself (64 KB per row of
    // V = 262,144 from L2, per tile): one launch fewer, and one per pass.
    const int fused = s.rows <= kSplitFuseRows ? 1 : 0;
    if (!fused) hipLaunchKernelGGL(fs_bitmap_kernel, rows, dim3(kSThreads), 0, stream, s);
    hipLaunchKernelGGL(fs_keys_kernel, tiles, dim3(kKThreads), 0, stream, s, fused);
    for (int pass = 0; pass < 4; ++pass) {
        const int src_is_buf1 = pass & 1;  // buf0 -> buf1 -> buf0 -> buf1 -> buf0
        if (pass > 0) hipLaunchKernelGGL(fs_count_kernel, tiles, dim3(kKThreads), 0, stream, s, 8 * pass, src_is_buf1);
        if (!fused) hipLaunchKernelGGL(fs_scan_kernel, rows, dim3(kSThreads), 0, stream, s, T);
        hipLaunchKernelGGL(fs_scatter_kernel, tiles, dim3(kKThreads), 0, stream, s, 8 * pass, src_is_buf1, fused);
    }
    hipLaunchKernelGGL(fs_bounds_kernel, tiles, dim3(kKThreads), 0, stream, s);
    hipLaunchKernelGGL(fs_istart_kernel, tiles, dim3(kKThreads), 0, stream, s);
    hipLaunchKernelGGL(fs_exps_kernel, tiles, dim3(kKThreads), 0, stream, s);
    hipLaunchKernelGGL(fs_meta_kernel, rows, dim3(64), 0, stream, s, T);
    return hipGetLastError();
}

template <typename T>
hipError_t sorted_pass(const DevArgs& a, hipStream_t stream) {
    const int64_t stride = fo_items_stride_f32(a.vocab);
    if (a.fo_capacity < stride) return hipErrorInvalidValue;
    const int64_t per64 = std::min<int64_t>(a.fo_capacity / stride, a.rows);
    // f32 slices of up to kSplitMaxRows rows take the many-workgroup sort
    // (when the handle's tile area holds them): its time grows with the rows,
    // while fo_sort_kernel runs up to 256 rows side by side in about the time
    // of one (about equal near 200 rows of V = 262,144). Not with per-row
    // parameters: the host cannot tell whether any row needs this path, and
    // the many-workgroup sort is 12 to 17 launches, about 30 µs even when every
    // row leaves at once, against two for fo_sort_kernel.
    const bool split = std::is_same<T, float>::value && !a.fo_fallback && a.fo_tiles != nullptr && !a.row_params &&
                       per64 <= kSplitMaxRows && per64 * fo_tile_words(fo_split_tiles(a.vocab)) <= a.fo_tiles_words;
    const int per = static_cast<int>(std::max<int64_t>(1, per64));
    // The denominator's tile maps go to the tile area when it holds a slice.
    const bool maps = a.fo_tiles != nullptr && map_row_words(a.vocab) <= fo_tile_words(fo_split_tiles(a.vocab)) &&
                      static_cast<int64_t>(per) * fo_tile_words(fo_split_tiles(a.vocab)) <= a.fo_tiles_words &&
                      per <= kMapRowGroups * 64 &&
                      (a.vocab + kMapTile - 1) / kMapTile * kMapSub * (kMapPartWords + 1) + 8 <= kFoExtrasCap;
    for (int r0 = 0; r0 < a.rows; r0 += per) {
        DevArgs s = slice_rows(a, r0, std::min(per, a.rows - r0));
        s.fo_items_stride = stride;
        if (split) {
            const hipError_t es = split_sort_f32(s, stream);
            if (es != hipSuccess) return es;
        } else {
            hipLaunchKernelGGL(fo_sort_kernel<T>, dim3(s.rows), dim3(kThreads), 0, stream, s);
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        s.fo_maps = 0;
        if (maps) {
            const int parts = (a.vocab + kMapTile - 1) / kMapTile * kMapSub;
            const int groups = std::min(s.rows, kMapRowGroups);
            hipLaunchKernelGGL(fo_denmap_kernel, dim3(parts, groups), dim3(kMapThreads), 0, stream, s);
            e = hipGetLastError();
            if (e != hipSuccess) return e;
            s.fo_maps = 1;
        }
        hipLaunchKernelGGL((fo_decide_kernel<T, true>), dim3(s.rows), dim3(kDThreads), 0, stream, s);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace

hipError_t launch_full_order(const DevArgs& a, hipStream_t stream, bool penalised_overflow) {
    if (!a.fo_items) return hipErrorInvalidValue;
    if (a.dtype == GE_DTYPE_BF16) {
        hipLaunchKernelGGL(fo_hist_kernel, dim3(a.rows), dim3(kThreads), 0, stream, a);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL((fo_decide_kernel<uint16_t, false>), dim3(a.rows), dim3(kDThreads), 0, stream, a);
        e = hipGetLastError();
        if (e != hipSuccess || !penalised_overflow) return e;
        // Rows flagged for too many unique penalised ids: sorted items, as
        // for f32 rows, then their draw again (the first pass wrote token -1
        // and left their ring and done state alone).
        DevArgs f = a;
        f.fo_fallback = 1;
        return sorted_pass<uint16_t>(f, stream);
    }
    return sorted_pass<float>(a, stream);
}

}  // namespace ge
