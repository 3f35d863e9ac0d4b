// gfx950 sampling kernels for the GemmaEdge token sampler.
//
// One launch samples `rows` rows. Each row is split into `cpr` chunks of
// kBlock * EPT logits, one workgroup per chunk. A workgroup
//   1. issues its chunk's 16-byte loads (consecutive threads on consecutive
//      addresses) and, while they are in flight, builds the chunk's penalty
//      bitmap in LDS from the row's history;
//   2. takes the maximum RAW logit of each group of EPT/GPT of its slots
//      (penalised tokens left out) and finds, with two adaptive 8-bit radix
//      digits over their order keys, a lower bound tau on the k-th largest of
//      those maxima: at least k non-penalised logits of the chunk are >= tau,
//      so softcap(tau) bounds the row's k-th largest final value from below;
//   3. lowers tau to the first raw key whose softcapped value equals
//      softcap(tau) (softcap is monotone, so this keeps every logit that could
//      tie after capping);
//   4. compacts its candidates into LDS — the non-penalised logits at or above
//      that floor, and its penalised tokens that could still reach the top-k —
//      evaluates their final values there (softcap, then the penalty: each
//      token once, so history duplicates cannot apply it twice), and publishes
//      them as (final value desc, index asc) composite keys;
//   5. takes a ticket; the last workgroup of the row merges the chunks' lists
//      (their union contains the row's top-k with exact final values), selects
//      and sorts the top-k and runs the reference's softmax / min-p / top-p /
//      draw in its exact operation order (src/generation.cpp:89-126).
//
// Cross-workgroup data (candidate lists and counts) is written with
// agent-scope relaxed atomic stores and read with agent-scope relaxed atomic
// loads. On gfx950 these are plain loads/stores with the sc1 bit, coherent
// across the XCDs' L2s; each wave waits for its stores (s_waitcnt) before the
// workgroup barrier that precedes the ticket. This avoids __threadfence(),
// which on this chip writes back and invalidates the XCD's whole L2.
//
// No MFMA: nothing here is a contraction. The bound is HBM bandwidth.
#include <hip/hip_runtime.h>

#include <climits>
#include <type_traits>

#include "ge_math.h"
#include "sampler_internal.h"

#pragma clang fp contract(off)

namespace ge {
namespace {

constexpr int kBatch = 8;     // independent global loads in flight per thread
constexpr int kPenCap = 1024; // penalised tokens of one chunk listed in LDS

template <typename U>
__device__ __forceinline__ void store_shared(U* p, U v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename U>
__device__ __forceinline__ U load_shared(const U* p) {
    return __hip_atomic_load(const_cast<U*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
    const int lane = __lane_id();
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t t = __shfl_up(v, d, 64);
        if (lane >= d) v += t;
    }
    return v;
}

__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v = max(v, static_cast<uint32_t>(__shfl_xor(v, d, 64)));
    return v;
}

__device__ __forceinline__ uint32_t wave_min(uint32_t v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v = min(v, static_cast<uint32_t>(__shfl_xor(v, d, 64)));
    return v;
}

__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v = min(v, __shfl_xor(v, d, 64));
    return v;
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
    return v;
}

__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
}

__device__ __forceinline__ float readlane_f(float v, int i) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
}

__device__ __forceinline__ double readlane_d(double v, int i) {
    const uint64_t b = d2u(v);
    const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(b), i);
    const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(b >> 32), i);
    return u2d((static_cast<uint64_t>(hi) << 32) | lo);
}

// Lane I of the result is `v` (a wave-uniform value); other lanes keep `old`.
// One v_writelane_b32 with an immediate lane index.
template <int I>
__device__ __forceinline__ uint32_t writelane_u(uint32_t v, uint32_t old) {
    const uint32_t s = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
    asm volatile("v_writelane_b32 %0, %1, %2" : "+v"(old) : "s"(s), "i"(I));
    return old;
}
template <int I>
__device__ __forceinline__ float writelane_f(float v, float old) {
    return u2f(writelane_u<I>(f2u(v), f2u(old)));
}
template <int I>
__device__ __forceinline__ double writelane_d(double v, double old) {
    const uint64_t b = d2u(v), o = d2u(old);
    const uint32_t lo = writelane_u<I>(static_cast<uint32_t>(b), static_cast<uint32_t>(o));
    const uint32_t hi = writelane_u<I>(static_cast<uint32_t>(b >> 32), static_cast<uint32_t>(o >> 32));
    return u2d((static_cast<uint64_t>(hi) << 32) | lo);
}

// Calls f(std::integral_constant<int, J>) for J = 0 .. N-1, in order.
template <int J, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (J < N) {
        f(std::integral_constant<int, J>{});
        static_for<J + 1, N>(f);
    }
}

__device__ __forceinline__ float load_one(const float* rowp, int i) { return rowp[i]; }
__device__ __forceinline__ float load_one(const uint16_t* rowp, int i) { return bf16_to_f32(rowp[i]); }

__device__ __forceinline__ ge_sample_params row_params(const DevArgs& a, int row) {
    return a.row_params ? a.row_params[row] : a.params;
}

__device__ __forceinline__ void row_history(const DevArgs& a, int row, const int32_t*& h, int& n) {
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

// Exponent of the lowest set bit of a positive finite float.
__device__ __forceinline__ int lsb_exponent(float e) {
    const uint32_t b = f2u(e);
    const uint32_t ex = b >> 23;
    const uint32_t man = b & 0x7fffffu;
    if (ex == 0) return -149 + __builtin_ctz(man);
    return static_cast<int>(ex) - 150 + __builtin_ctz(man | 0x800000u);
}

struct Shared {
    union {
        uint64_t surv[kSurvivorCap];  // merge: union cache, then survivors (composite keys)
        struct {
            uint32_t raw[kSurvivorCap];  // streaming pass: candidate logit bits
            uint32_t tag[kSurvivorCap];  // streaming pass: token index
        } stage;
    };
    uint32_t pen_idx[kPenCap];  // streaming pass: the chunk's penalised tokens...
    uint32_t pen_raw[kPenCap];  // ...and their raw logit bits
    float prob[kMaxTopK];
    uint32_t hist[256];
    uint32_t off[kMaxChunks + 1];  // exclusive prefix of the chunks' candidate counts
    double f64[kBlock / 64];
    int i32[kBlock / 64];
    uint32_t u32[32];
};

// Exclusive prefix over the workgroup of one value per thread; also returns
// the total. Uses sh.u32[24..28]; contains barriers (block-uniform).
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t& total, Shared& sh) {
    const int lane = __lane_id();
    const int wave = threadIdx.x >> 6;
    const uint32_t incl = wave_incl_scan(v);
    if (lane == 63) sh.u32[24 + wave] = incl;
    __syncthreads();
    uint32_t before = 0;
    for (int w = 0; w < wave; ++w) before += sh.u32[24 + w];
    total = sh.u32[24] + sh.u32[25] + sh.u32[26] + sh.u32[27];
    __syncthreads();
    return before + incl - v;
}

// Wave 0: hist[256] holds counts per digit; find the digit b (scanning from
// 255 down) where the running count first reaches k. Writes b, the count above
// b, and whether the total is below k.
__device__ __forceinline__ void find_bin_desc(const uint32_t* hist, uint32_t k, uint32_t* out) {
    const int lane = __lane_id();
    const int b0 = 255 - 4 * lane;
    uint32_t h[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) h[i] = hist[b0 - i];
    const uint32_t s = h[0] + h[1] + h[2] + h[3];
    const uint32_t incl = wave_incl_scan(s);
    const uint32_t total = __shfl(incl, 63, 64);
    if (total < k) {
        if (lane == 0) {
            out[0] = 0;
            out[1] = 0;
            out[2] = 1;
        }
        return;
    }
    uint32_t c = incl - s;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (c < k && c + h[i] >= k) {
            out[0] = static_cast<uint32_t>(b0 - i);
            out[1] = c;
            out[2] = 0;
        }
        c += h[i];
    }
}

// Lower bound on the k-th largest of the keys that `visit` presents within
// [lo, hi] (every thread calls visit(f) and f(key) runs once per key it
// holds). Two radix passes over the 8-bit digits right below the common prefix
// of lo and hi, so the keys spread over the bins. Returns 0 if fewer than k
// keys lie in [lo, hi]. Uses sh.hist and sh.u32[20..22]; block-uniform.
template <typename Visit>
__device__ __forceinline__ uint32_t block_kth(uint32_t lo, uint32_t hi, uint32_t k, Visit&& visit,
                                              Shared& sh) {
    const int tid = threadIdx.x;
    if (lo > hi || k == 0) return 0u;
    const uint32_t diff = lo ^ hi;
    const int common = diff ? __clz(static_cast<int>(diff)) : 32;
    const int shift1 = max(32 - common - 8, 0);
    const uint32_t base1 = lo >> shift1;
    for (int i = tid; i < 256; i += kBlock) sh.hist[i] = 0u;
    __syncthreads();
    visit([&](uint32_t key) {
        if (key >= lo && key <= hi) atomicAdd(&sh.hist[(key >> shift1) - base1], 1u);
    });
    __syncthreads();
    if (tid < 64) find_bin_desc(sh.hist, k, &sh.u32[20]);
    __syncthreads();
    const uint32_t d1 = sh.u32[20];
    const uint32_t above = sh.u32[21];
    const bool short_set = sh.u32[22] != 0u;
    __syncthreads();
    if (short_set) return 0u;
    const uint32_t pre = base1 + d1;
    if (shift1 == 0) return pre;
    const int shift2 = max(shift1 - 8, 0);
    const uint32_t bucket = pre << shift1;
    for (int i = tid; i < 256; i += kBlock) sh.hist[i] = 0u;
    __syncthreads();
    visit([&](uint32_t key) {
        if (key >= lo && key <= hi && (key >> shift1) == pre)
            atomicAdd(&sh.hist[(key - bucket) >> shift2], 1u);
    });
    __syncthreads();
    if (tid < 64) find_bin_desc(sh.hist, k - above, &sh.u32[20]);
    __syncthreads();
    const uint32_t d2 = sh.u32[20];
    __syncthreads();
    return bucket + (d2 << shift2);
}

// Called by one whole wave; every lane returns the same value: the smallest
// raw key x <= tau with softcap(x) == softcap(tau). softcap is monotone
// non-decreasing (glibc tanhf is monotone on all floats), so the keys with
// equal capped value form an interval. Usually tau-1 already caps lower and
// one evaluation round decides; otherwise a 64-way search finds the floor.
__device__ __forceinline__ uint32_t tie_floor(uint32_t tau, float cap) {
    if (!(cap > 0.0f) || tau <= kKeyNegInf) return tau;
    const int lane = __lane_id();
    const float s01 = softcap(key_value(tau - static_cast<uint32_t>(lane & 1)), cap);
    const float target = __shfl(s01, 0, 64);
    if (__shfl(s01, 1, 64) != target) return tau;
    uint32_t hi = tau - 1;  // lowest key known to map to target
    uint32_t lo;            // a key known to map below target
    uint64_t step = 1;
    for (;;) {
        const uint64_t off = static_cast<uint64_t>(lane + 1) * step;
        const uint32_t x = (static_cast<uint64_t>(hi - kKeyNegInf) > off)
                               ? hi - static_cast<uint32_t>(off)
                               : kKeyNegInf;
        const bool eq = softcap(key_value(x), cap) == target;
        const uint64_t ne = __ballot(!eq);
        if (ne) {
            const int j = __ffsll(static_cast<unsigned long long>(ne)) - 1;
            const uint32_t xj = __shfl(x, j, 64);
            const uint32_t xp = __shfl(x, j > 0 ? j - 1 : 0, 64);
            lo = xj;
            hi = j > 0 ? xp : hi;
            break;
        }
        hi = __shfl(x, 63, 64);
        if (hi == kKeyNegInf) return kKeyNegInf;
        step *= 64;
    }
    while (hi - lo > 1) {
        const uint32_t span = hi - lo;
        const uint32_t s = (span + 63u) / 64u;
        const uint64_t off = static_cast<uint64_t>(lane + 1) * s;
        const uint32_t x = off < span ? lo + static_cast<uint32_t>(off) : hi;
        const bool eq = softcap(key_value(x), cap) == target;
        const uint64_t m = __ballot(eq);  // non-empty: lanes probing hi match
        const int j = __ffsll(static_cast<unsigned long long>(m)) - 1;
        const uint32_t xj = __shfl(x, j, 64);
        const uint32_t xp = __shfl(x, j > 0 ? j - 1 : 0, 64);
        lo = j > 0 ? xp : lo;
        hi = xj;
    }
    return hi;
}

// Descending bitonic sort of s[0, n), n a power of two <= kSurvivorCap, by the
// whole workgroup through LDS.
__device__ __forceinline__ void bitonic_desc_block(uint64_t* s, uint32_t n) {
    const int tid = threadIdx.x;
    for (uint32_t size = 2; size <= n; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t i = tid; i < n / 2; i += kBlock) {
                const uint32_t pos = 2 * i - (i & (stride - 1));
                const uint32_t q = pos + stride;
                const bool desc = (pos & size) == 0;
                const uint64_t x = s[pos], y = s[q];
                if ((x < y) == desc) {
                    s[pos] = y;
                    s[q] = x;
                }
            }
            __syncthreads();
        }
    }
}

// Descending bitonic sort of 64 values, one per lane, within one wave.
__device__ __forceinline__ uint64_t bitonic_desc_wave(uint64_t x) {
    const uint32_t lane = __lane_id();
#pragma unroll
    for (uint32_t size = 2; size <= 64; size <<= 1) {
#pragma unroll
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            const uint64_t y = __shfl_xor(x, static_cast<int>(stride), 64);
            const bool lower = (lane & stride) == 0;
            const bool desc = (lane & size) == 0 || size == 64;
            x = (lower == desc) ? (x > y ? x : y) : (x < y ? x : y);
        }
    }
    return x;
}

// Descending bitonic sort of 64 keys, one per lane, within one wave.
__device__ __forceinline__ uint32_t bitonic_desc_wave_u32(uint32_t x) {
    const uint32_t lane = __lane_id();
#pragma unroll
    for (uint32_t size = 2; size <= 64; size <<= 1) {
#pragma unroll
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            const uint32_t y = static_cast<uint32_t>(__shfl_xor(static_cast<int>(x), static_cast<int>(stride), 64));
            const bool lower = (lane & stride) == 0;
            const bool desc = (lane & size) == 0 || size == 64;
            x = (lower == desc) ? max(x, y) : min(x, y);
        }
    }
    return x;
}

// Visits every entry of the row's candidate union [0, total) in global memory
// with kBatch agent-coherent loads in flight per thread. off[] (LDS) is the
// exclusive prefix of the per-chunk counts; entry g lives in the chunk c with
// off[c] <= g < off[c+1]. f(g, entry) runs for each entry.
template <typename F>
__device__ __forceinline__ void walk_union(const uint64_t* cand_row, int chunk_len, const uint32_t* off,
                                           int cpr, uint32_t total, F&& f) {
    for (uint32_t base = 0; base < total; base += kBlock * kBatch) {
        uint64_t e[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const uint32_t g = base + u * kBlock + threadIdx.x;
            e[u] = 0ull;
            if (g < total) {
                int lo = 0, hi = cpr;
                while (hi - lo > 1) {
                    const int mid = (lo + hi) >> 1;
                    if (off[mid] <= g) lo = mid;
                    else hi = mid;
                }
                e[u] = load_shared(&cand_row[static_cast<int64_t>(lo) * chunk_len + (g - off[lo])]);
            }
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const uint32_t g = base + u * kBlock + threadIdx.x;
            if (g < total) f(g, e[u]);
        }
    }
}

__device__ __forceinline__ void write_row(const DevArgs& a, int row, int32_t token, float prob,
                                          int32_t flags) {
    a.tokens[row] = token;
    if (a.probs) a.probs[row] = prob;
    if (a.flags) a.flags[row] = flags;
    if (a.ring) {
        const uint32_t len = static_cast<uint32_t>(a.ring_len[row]);
        a.ring[static_cast<int64_t>(row) * a.ring_capacity +
               static_cast<int64_t>(len % static_cast<uint32_t>(a.ring_capacity))] = token;
        a.ring_len[row] = static_cast<int32_t>(len + 1u);
    }
    a.tickets[row] = 0u;  // ready for the next launch
}

// generation.cpp:103-126 on probabilities sorted by value desc / index asc,
// evaluated by one whole wave. seg_prob(g) returns this lane's probability of
// entry g * 64 + lane (0 past keff). The reference's cumulative sums are
// sequential fp32 (and, for the boundary distances, double) chains: every lane
// computes the same chain and lane j keeps step j of each 64-entry segment, so
// each stop test is one ballot rather than a branch per step.
template <typename P>
__device__ __forceinline__ void scan_and_walk(P&& seg_prob, uint32_t keff, const ge_sample_params& p,
                                              float u, uint32_t& pos_out, bool& near_out) {
    const int lane = __lane_id();
    const float minimum = readlane_f(seg_prob(0u), 0) * p.min_p;
    // min-p / top-p cut (generation.cpp:103-115).
    float cum = 0.0f;
    float mass = 0.0f;
    uint32_t keep = keff;
    bool stopped = false;
    const uint32_t nseg = (keff + 63) / 64;
    for (uint32_t g = 0; g < nseg && !stopped; ++g) {
        const float pl = seg_prob(g);
        const float before = cum;
        float cl = 0.0f;
        static_for<0, 64>([&](auto J) {
            cum = cum + readlane_f(pl, J);
            cl = writelane_f<J>(cum, cl);
        });
        const uint32_t idx = g * 64 + static_cast<uint32_t>(lane);
        const bool valid = idx < keff && idx > 0;
        const uint64_t mh = __ballot(valid && pl < minimum);     // checked before adding
        const uint64_t th = __ballot(valid && cl >= p.top_p);    // checked after adding
        if (mh | th) {
            const int jm = mh ? __ffsll(static_cast<unsigned long long>(mh)) - 1 : 64;
            const int jt = th ? __ffsll(static_cast<unsigned long long>(th)) - 1 : 64;
            if (jm <= jt) {
                keep = g * 64 + static_cast<uint32_t>(jm);
                mass = jm > 0 ? readlane_f(cl, jm - 1) : before;
            } else {
                keep = g * 64 + static_cast<uint32_t>(jt) + 1;
                mass = readlane_f(cl, jt);
            }
            stopped = true;
        }
    }
    // The reference's `mass` loop (generation.cpp:117-118) adds the same probs
    // in the same order from 0, so it equals the cumulative sum at the cut.
    if (!stopped) mass = cum;  // entries past keff add exact zeros
    const float choice0 = u * mass + 0.0f;  // uniform_real_distribution(0, mass)
    // Subtract walk (generation.cpp:120-126) with the CDF boundaries around it.
    float choice = choice0;
    double dc = 0.0;
    uint32_t pos = keep - 1;
    double c_before = 0.0, c_at = 0.0;
    bool found = false;
    const uint32_t nseg2 = (keep + 63) / 64;
    for (uint32_t g = 0; g < nseg2 && !found; ++g) {
        const float pl = seg_prob(g);
        const double dbefore = dc;
        float chl = 0.0f;
        double dl = 0.0;
        static_for<0, 64>([&](auto J) {
            const float pj = readlane_f(pl, J);
            choice = choice - pj;
            dc = dc + static_cast<double>(pj);
            chl = writelane_f<J>(choice, chl);
            dl = writelane_d<J>(dc, dl);
        });
        const uint32_t idx = g * 64 + static_cast<uint32_t>(lane);
        const uint64_t hit = __ballot(idx < keep && chl <= 0.0f);
        int j = -1;
        if (hit) {
            j = __ffsll(static_cast<unsigned long long>(hit)) - 1;
            pos = g * 64 + static_cast<uint32_t>(j);
            found = true;
        } else if (g == nseg2 - 1) {
            j = static_cast<int>(keep - 1 - g * 64);  // fallthrough return, generation.cpp:126
        }
        if (j >= 0) {
            c_at = readlane_d(dl, j);
            c_before = j > 0 ? readlane_d(dl, j - 1) : dbefore;
        }
    }
    bool near = false;
    if (pos > 0 && fabs(static_cast<double>(choice0) - c_before) < 1e-6) near = true;
    if (pos + 1 < keep && fabs(static_cast<double>(choice0) - c_at) < 1e-6) near = true;
    pos_out = pos;
    near_out = near;
}

// std::max_element (generation.cpp:66-70) keeps index 0 when its value is NaN
// (NaN < x is false), so greedy returns 0 then. Token 0's final value is NaN
// iff its raw value is, unless the penalty itself is NaN and 0 is in history.
template <typename T>
__device__ __forceinline__ bool final0_is_nan(const T* rowp, float cap, bool pen, float r,
                                              const int32_t* hist, int H) {
    if (__builtin_isnan(softcap(load_one(rowp, 0), cap))) return true;
    if (!pen || !__builtin_isnan(r)) return false;
    for (int j = 0; j < H; ++j)
        if (hist[j] == 0) return true;
    return false;
}

template <typename T>
__device__ __forceinline__ void merge_row(const DevArgs& a, Shared& sh, int row,
                                          const ge_sample_params& p, bool greedy, uint32_t k,
                                          const T* rowp, const int32_t* hist, int H, bool pen,
                                          int chunk_len) {
    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int wave = tid >> 6;
    const uint64_t* cand_row = a.cand + static_cast<int64_t>(row) * a.cand_stride;

    // Chunk counts -> exclusive prefix in LDS.
    const uint32_t cnt = tid < a.cpr ? load_shared(&a.chunk_count[row * kMaxChunks + tid]) : 0u;
    uint32_t total;
    const uint32_t excl = block_excl_scan(cnt, total, sh);
    if (tid < a.cpr) sh.off[tid] = excl;
    if (tid == 0) {
        sh.off[a.cpr] = total;
        sh.u32[16] = 0u;           // max final key
        sh.u32[17] = 0xffffffffu;  // min final key
        sh.u32[3] = 0u;            // survivors
    }
    __syncthreads();
    const bool cached = total <= static_cast<uint32_t>(kSurvivorCap);

    // One pass over the union (composite keys of final values): cache it in
    // LDS when it fits, and the range of its final keys.
    uint32_t kmax = 0, kmin = 0xffffffffu;
    walk_union(cand_row, chunk_len, sh.off, a.cpr, total, [&](uint32_t g, uint64_t e) {
        const uint32_t key = composite_key(e);
        kmax = max(kmax, key);
        kmin = min(kmin, key);
        if (cached) sh.surv[g] = e;
    });
    kmax = wave_max(kmax);
    kmin = wave_min(kmin);
    if (lane == 0) {
        atomicMax(&sh.u32[16], kmax);
        atomicMin(&sh.u32[17], kmin);
    }
    __syncthreads();

    // The union holds the row's top-k (by final value, then index); the k-th
    // largest final key bounds the survivors.
    auto visit_union = [&](auto&& f) {
        if (cached) {
            for (uint32_t g = tid; g < total; g += kBlock) f(composite_key(sh.surv[g]));
        } else {
            walk_union(cand_row, chunk_len, sh.off, a.cpr, total,
                       [&](uint32_t, uint64_t e) { f(composite_key(e)); });
        }
    };
    const uint32_t kfloor = total > k ? block_kth(sh.u32[17], sh.u32[16], k, visit_union, sh) : 0u;

    if (cached) {
        // Compact the survivors to the front of the cache (read first: the
        // survivor list overwrites it).
        constexpr int kPer = kSurvivorCap / kBlock;
        uint64_t e[kPer];
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const uint32_t g = u * kBlock + tid;
            e[u] = g < total ? sh.surv[g] : 0ull;
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const uint32_t g = u * kBlock + tid;
            if (g < total && composite_key(e[u]) >= kfloor) sh.surv[atomicAdd(&sh.u32[3], 1u)] = e[u];
        }
    } else {
        walk_union(cand_row, chunk_len, sh.off, a.cpr, total, [&](uint32_t, uint64_t e) {
            if (composite_key(e) >= kfloor) {
                const uint32_t pos = atomicAdd(&sh.u32[3], 1u);
                if (pos < kSurvivorCap) sh.surv[pos] = e;
            }
        });
    }
    __syncthreads();
    const uint32_t nsurv = sh.u32[3];

    if (nsurv == 0 || nsurv > kSurvivorCap) {
        // More survivors than LDS holds (massive exact ties) or none at all.
        if (tid == 0) write_row(a, row, -1, 0.0f, GE_FLAG_UNSUPPORTED);
        return;
    }
    const uint32_t keff = min(k, nsurv);
    const float u = greedy ? 0.0f : a.uniforms[row];
    const float r = p.repetition_penalty;

    if (nsurv <= 64) {
        // One wave: sort in registers, softmax and the sequential scans with
        // lane-resident probabilities (no barriers).
        if (wave != 0) return;
        const uint64_t c = bitonic_desc_wave(lane < static_cast<int>(nsurv) ? sh.surv[lane] : 0ull);
        if (greedy) {
            int32_t token = static_cast<int32_t>(composite_index(__shfl(c, 0, 64)));
            if (lane == 0) {
                if (final0_is_nan(rowp, p.softcap, pen, r, hist, H)) token = 0;
                write_row(a, row, token, 1.0f, 0);
            }
            return;
        }
        // generation.cpp:89-101 — p_i = expf((v_i - max) * (1/T)); double denominator.
        const float maximum = key_value(composite_key(__shfl(c, 0, 64)));
        const float inv_temp = 1.0f / p.temperature;
        const bool live = lane < static_cast<int>(keff);
        const float e = live ? expf_glibc((key_value(composite_key(c)) - maximum) * inv_temp) : 0.0f;
        const bool bad = live && (!(e >= 0.0f) || __builtin_isinf(e));
        const int lsb = (live && e > 0.0f && !bad) ? lsb_exponent(e) : INT_MAX;
        const double s = wave_sum(static_cast<double>(e));
        const int m = wave_min_i(lsb);
        const int ex = static_cast<int>((d2u(s) >> 52) & 0x7ffu) - 1023;
        double den;
        if (!__any(bad) && s > 0.0 && !__builtin_isinf(s) && m >= ex - 51) {
            den = s;  // certified exact, as in the workgroup path below
        } else {
            den = 0.0;
            for (uint32_t i = 0; i < keff; ++i) den += static_cast<double>(readlane_f(e, static_cast<int>(i)));
        }
        const float inv_denom = static_cast<float>(1.0 / den);
        const float pr = e * inv_denom;
        uint32_t pos;
        bool near;
        scan_and_walk([&](uint32_t) { return pr; }, keff, p, u, pos, near);
        const int32_t token = static_cast<int32_t>(composite_index(__shfl(c, static_cast<int>(pos), 64)));
        const float prob = readlane_f(pr, static_cast<int>(pos));
        if (lane == 0) write_row(a, row, token, prob, near ? GE_FLAG_NEAR_BOUNDARY : 0);
        return;
    }

    uint32_t n2 = 1;
    while (n2 < nsurv) n2 <<= 1;
    for (uint32_t i = nsurv + tid; i < n2; i += kBlock) sh.surv[i] = 0ull;
    __syncthreads();
    bitonic_desc_block(sh.surv, n2);

    if (greedy) {
        if (tid == 0) {
            int32_t token = static_cast<int32_t>(composite_index(sh.surv[0]));
            if (final0_is_nan(rowp, p.softcap, pen, r, hist, H)) token = 0;
            write_row(a, row, token, 1.0f, 0);
        }
        return;
    }
    // generation.cpp:89-101 — p_i = expf((v_i - max) * (1/T)); double denominator.
    const float maximum = key_value(composite_key(sh.surv[0]));
    const float inv_temp = 1.0f / p.temperature;
    double lsum = 0.0;
    int lmin = INT_MAX;
    int bad = 0;
    for (uint32_t i = tid; i < keff; i += kBlock) {
        const float v = key_value(composite_key(sh.surv[i]));
        const float e = expf_glibc((v - maximum) * inv_temp);
        sh.prob[i] = e;
        lsum += static_cast<double>(e);
        if (!(e >= 0.0f) || __builtin_isinf(e)) bad = 1;
        else if (e > 0.0f) lmin = min(lmin, lsb_exponent(e));
    }
    lsum = wave_sum(lsum);
    lmin = wave_min_i(lmin);
    bad = __any(bad);
    if (lane == 0) {
        sh.f64[wave] = lsum;
        sh.i32[wave] = bad ? INT_MIN : lmin;
    }
    __syncthreads();
    if (tid == 0) {
        double s = 0.0;
        int m = INT_MAX;
        bool b = false;
        for (int w = 0; w < kBlock / 64; ++w) {
            s += sh.f64[w];
            if (sh.i32[w] == INT_MIN) b = true;
            else m = min(m, sh.i32[w]);
        }
        // Certified exact: every term is a multiple of 2^m and every partial
        // sum is below 2^(E+2), so 53 bits hold each partial sum exactly when
        // m >= E - 51; then any summation order equals the reference's
        // sequential one. Otherwise replay it sequentially.
        double den;
        int ex = 0;
        if (!b && s > 0.0 && !__builtin_isinf(s)) ex = static_cast<int>((d2u(s) >> 52) & 0x7ffu) - 1023;
        if (!b && s > 0.0 && !__builtin_isinf(s) && m >= ex - 51) {
            den = s;
        } else {
            den = 0.0;
            for (uint32_t i = 0; i < keff; ++i) den += static_cast<double>(sh.prob[i]);
        }
        sh.f64[0] = den;
    }
    __syncthreads();
    const float inv_denom = static_cast<float>(1.0 / sh.f64[0]);
    for (uint32_t i = tid; i < keff; i += kBlock) sh.prob[i] = sh.prob[i] * inv_denom;
    __syncthreads();
    if (wave == 0) {
        uint32_t pos;
        bool near;
        scan_and_walk(
            [&](uint32_t g) {
                const uint32_t i = g * 64 + static_cast<uint32_t>(lane);
                return i < keff ? sh.prob[i] : 0.0f;
            },
            keff, p, u, pos, near);
        if (lane == 0)
            write_row(a, row, static_cast<int32_t>(composite_index(sh.surv[pos])), sh.prob[pos],
                      near ? GE_FLAG_NEAR_BOUNDARY : 0);
    }
}

template <typename T, int EPT, int GPT>
__global__ __launch_bounds__(kBlock) void select_kernel(DevArgs a) {
    constexpr int W = sizeof(T) == 4 ? 4 : 8;  // elements per 16-byte load
    constexpr int NV = EPT / W;                 // 16-byte loads per thread
    constexpr int NW = EPT * sizeof(T) / 4;     // 32-bit words per thread
    constexpr int CHUNK = kBlock * EPT;
    constexpr int GSZ = EPT / GPT;
    static_assert(EPT % W == 0 && EPT % GPT == 0 && EPT <= 64, "bad tiling");

    __shared__ uint32_t s_pbits[CHUNK / 32];
    __shared__ Shared sh;

    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int wave = tid >> 6;
    const int row = blockIdx.x / a.cpr;
    const int chunk = blockIdx.x - row * a.cpr;
    const int V = a.vocab;
    const ge_sample_params p = row_params(a, row);
    const bool greedy = p.temperature <= 0.0f;  // generation.cpp:66
    const uint32_t k = greedy ? 1u
                              : (p.top_k ? min(p.top_k, static_cast<uint32_t>(V))
                                         : static_cast<uint32_t>(V));  // generation.cpp:80
    if (k > static_cast<uint32_t>(kMaxTopK)) {
        // bf16 rows belong to the full-order kernels, which the host launches
        // whenever the handle has their workspace.
        if (a.dtype == GE_DTYPE_BF16 && a.fo_items) return;
        if (chunk == 0 && tid == 0) {
            a.tokens[row] = -1;
            if (a.probs) a.probs[row] = 0.0f;
            if (a.flags) a.flags[row] = GE_FLAG_UNSUPPORTED;
        }
        return;
    }
    const T* rowp = static_cast<const T*>(a.logits) + static_cast<int64_t>(row) * a.row_stride;
    const int32_t* hist;
    int H;
    row_history(a, row, hist, H);
    const float r = p.repetition_penalty;
    const bool pen = H > 0 && !(r == 1.0f);
    const float cap = p.softcap;
    const int c0 = chunk * CHUNK;
    const int cend = min(c0 + CHUNK, V);

    // Slot s of this thread is element c0 + ((s / W) * kBlock + tid) * W + s % W.
    auto elem = [&](int s) { return c0 + ((s / W) * kBlock + tid) * W + (s % W); };
    constexpr uint32_t kHole = 0x7fc00000u;  // NaN placed in penalised / out-of-range slots

    // 1. Issue the chunk's loads first so their latency overlaps the bitmap build.
    uint32_t d[NW];
    if (a.vec_ok && c0 + CHUNK <= V) {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const uint4 q = *reinterpret_cast<const uint4*>(rowp + c0 + (v * kBlock + tid) * W);
            d[4 * v + 0] = q.x;
            d[4 * v + 1] = q.y;
            d[4 * v + 2] = q.z;
            d[4 * v + 3] = q.w;
        }
    } else {
#pragma unroll
        for (int s = 0; s < EPT; ++s) {
            const int e = elem(s);
            const uint32_t bits = e < cend ? f2u(load_one(rowp, e)) : kHole;
            if constexpr (W == 4) {
                d[s] = bits;
            } else if (s % 2 == 0) {
                d[s / 2] = bits >> 16;
            } else {
                d[s / 2] |= bits & 0xffff0000u;
            }
        }
    }
    auto value = [&](int s) -> float {
        if constexpr (W == 4) return u2f(d[s]);
        else return u2f((s % 2 == 0) ? (d[s / 2] << 16) : (d[s / 2] & 0xffff0000u));
    };

    // 2. Penalty bitmap of this chunk (history loads kBatch-wide); penalised
    //    slots become holes: fmax and ">= floor" below never select a NaN.
    if (pen) {
        for (int w = tid; w < CHUNK / 32; w += kBlock) s_pbits[w] = 0u;
        if (tid == 0) sh.u32[5] = 0u;
        __syncthreads();
        for (int base = 0; base < H; base += kBlock * kBatch) {
            int t[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int j = base + u * kBlock + tid;
                t[u] = j < H ? hist[j] : -1;
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                if (t[u] >= c0 && t[u] < cend)
                    atomicOr(&s_pbits[(t[u] - c0) >> 5], 1u << ((t[u] - c0) & 31));
        }
        __syncthreads();
        // Each penalised slot is visited once here, so listing it dedupes the
        // history; the list keeps the raw value for the final evaluation.
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int li = (v * kBlock + tid) * W;  // W divides 32: one bitmap word
            const uint32_t bits = (s_pbits[li >> 5] >> (li & 31)) & ((1u << W) - 1u);
            if (bits) {
#pragma unroll
                for (int j = 0; j < W; ++j) {
                    if ((bits >> j) & 1u) {
                        const uint32_t pos = atomicAdd(&sh.u32[5], 1u);
                        if (pos < static_cast<uint32_t>(kPenCap)) {
                            sh.pen_idx[pos] = static_cast<uint32_t>(elem(v * W + j));
                            sh.pen_raw[pos] = f2u(value(v * W + j));
                        }
                        if constexpr (W == 4) d[4 * v + j] = kHole;
                        else if (j % 2 == 0) d[4 * v + j / 2] = (d[4 * v + j / 2] & 0xffff0000u) | (kHole >> 16);
                        else d[4 * v + j / 2] = (d[4 * v + j / 2] & 0xffffu) | (kHole & 0xffff0000u);
                    }
                }
            }
        }
    }

    // 3. Group maxima of the raw values (holes ignored) and the chunk bound tau
    //    over their order keys.
    uint32_t gkey[GPT];
    uint32_t gmx = 0, gmn = 0xffffffffu;
#pragma unroll
    for (int g = 0; g < GPT; ++g) {
        float m = value(g * GSZ);
#pragma unroll
        for (int j = 1; j < GSZ; ++j) m = fmaxf(m, value(g * GSZ + j));
        gkey[g] = order_key(m);
        gmx = max(gmx, gkey[g]);
        gmn = min(gmn, gkey[g]);
    }
    gmx = wave_max(gmx);
    gmn = wave_min(gmn);
    if (lane == 0) {
        sh.u32[8 + wave] = gmx;
        sh.u32[12 + wave] = gmn;
    }
    __syncthreads();
    const uint32_t bmax = max(max(sh.u32[8], sh.u32[9]), max(sh.u32[10], sh.u32[11]));
    const uint32_t bmin = min(min(sh.u32[12], sh.u32[13]), min(sh.u32[14], sh.u32[15]));
    uint32_t tau;
    if (k == 1) {
        tau = bmax;
    } else if (GPT == 1 && k <= 64) {
        // Each wave: the ceil(k/4)-th largest of its 64 group maxima; the
        // smallest of the four still leaves >= k maxima at or above it.
        const uint32_t srt = bitonic_desc_wave_u32(gkey[0]);
        const uint32_t tw = __shfl(srt, static_cast<int>((k + 3) / 4) - 1, 64);
        if (lane == 0) sh.u32[16 + wave] = tw;
        __syncthreads();
        tau = min(min(sh.u32[16], sh.u32[17]), min(sh.u32[18], sh.u32[19]));
    } else {
        tau = block_kth(bmin, bmax, k,
                        [&](auto&& f) {
#pragma unroll
                            for (int g = 0; g < GPT; ++g) f(gkey[g]);
                        },
                        sh);
    }

    // 4. Tie floor. A floor at or below kKeyNaN means "no pruning": fewer than
    //    k real non-penalised logits are known, so every slot is a candidate
    //    (NaN logits included, they sort last).
    if (wave == 0) {
        const uint32_t t = tie_floor(tau, cap);
        if (lane == 0) sh.u32[7] = max(t, kKeyNaN);
    }
    __syncthreads();
    const uint32_t thr = sh.u32[7];
    const bool allpass = thr <= kKeyNaN;
    const float floor_v = key_value(max(thr, kKeyNegInf));  // raw >= floor_v <=> key >= thr
    uint64_t cmask = 0;  // non-penalised candidate slots
    if (!allpass) {
#pragma unroll
        for (int s = 0; s < EPT; ++s) cmask |= static_cast<uint64_t>(value(s) >= floor_v) << s;
    } else {
#pragma unroll
        for (int s = 0; s < EPT; ++s) {
            const int e = elem(s);
            bool c = e < cend;
            if (c && pen) c = !((s_pbits[(e - c0) >> 5] >> ((e - c0) & 31)) & 1u);
            cmask |= static_cast<uint64_t>(c) << s;
        }
    }

    // 5. Compact the candidates into LDS (wave ballots, one region per wave),
    //    evaluate final values there, publish.
    uint32_t n_chunk;
    const uint32_t wfirst = block_excl_scan(
        __shfl(wave_incl_scan(static_cast<uint32_t>(__popcll(cmask))), 63, 64) * (lane == 63 ? 1u : 0u),
        n_chunk, sh);
    const uint32_t wave_base = __shfl(wfirst, 63, 64);
    uint64_t* region = a.cand + static_cast<int64_t>(row) * a.cand_stride + static_cast<int64_t>(c0);
    for (uint32_t base = 0; base < n_chunk; base += kSurvivorCap) {
        // Opaque per round: stops the compiler from hoisting 64 slot tests and
        // element indices out of this (nearly always single-trip) loop, which
        // would hold them all in registers.
        uint32_t cm_lo = static_cast<uint32_t>(cmask), cm_hi = static_cast<uint32_t>(cmask >> 32);
        int ebase = c0 + tid * W;
        asm volatile("" : "+v"(cm_lo), "+v"(cm_hi), "+v"(ebase));
        const uint64_t cm = (static_cast<uint64_t>(cm_hi) << 32) | cm_lo;
        uint32_t wb = wave_base;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const uint32_t vbits = static_cast<uint32_t>(cm >> (v * W)) & ((1u << W) - 1u);
            if (__ballot(vbits != 0u) == 0ull) continue;
#pragma unroll
            for (int j = 0; j < W; ++j) {
                const int s = v * W + j;
                const bool c = (vbits >> j) & 1u;
                const uint64_t m = __ballot(c);
                if (m) {
                    const uint32_t o = wb + lanes_below(m);
                    if (c && o >= base && o < base + kSurvivorCap) {
                        sh.stage.raw[o - base] = f2u(value(s));
                        sh.stage.tag[o - base] = static_cast<uint32_t>(ebase + v * kBlock * W + j);
                    }
                    wb += static_cast<uint32_t>(__popcll(m));
                }
            }
        }
        __syncthreads();
        const uint32_t n = min(n_chunk - base, static_cast<uint32_t>(kSurvivorCap));
        for (uint32_t i = tid; i < n; i += kBlock)
            store_shared(&region[base + i],
                         composite(order_key(softcap(u2f(sh.stage.raw[i]), cap)), sh.stage.tag[i]));
        __syncthreads();
    }

    // Penalised tokens of the chunk, from the LDS list (or, if it overflowed,
    // by claiming each in-range history id once: the thread whose atomicAnd
    // clears its bit owns it). With r >= 1 the penalty never raises a value, so
    // raw values below the floor cannot reach the top-k.
    if (pen) {
        if (tid == 0) sh.u32[6] = n_chunk;
        __syncthreads();
        const bool prune = r >= 1.0f && !allpass;
        const uint32_t npen = sh.u32[5];
        auto emit = [&](uint32_t t, float raw) {
            if (prune && !(raw >= floor_v)) return;
            const float f = penalize(softcap(raw, cap), r);
            store_shared(&region[atomicAdd(&sh.u32[6], 1u)], composite(order_key(f), t));
        };
        if (npen <= static_cast<uint32_t>(kPenCap)) {
            for (uint32_t i = tid; i < npen; i += kBlock) emit(sh.pen_idx[i], u2f(sh.pen_raw[i]));
        } else {
            for (int base = 0; base < H; base += kBlock * kBatch) {
                int t[kBatch];
#pragma unroll
                for (int u = 0; u < kBatch; ++u) {
                    const int j = base + u * kBlock + tid;
                    t[u] = j < H ? hist[j] : -1;
                }
#pragma unroll
                for (int u = 0; u < kBatch; ++u) {
                    if (t[u] >= c0 && t[u] < cend) {
                        const uint32_t bit = 1u << ((t[u] - c0) & 31);
                        if (!(atomicAnd(&s_pbits[(t[u] - c0) >> 5], ~bit) & bit)) t[u] = -1;
                    } else {
                        t[u] = -1;
                    }
                }
#pragma unroll
                for (int u = 0; u < kBatch; ++u)
                    if (t[u] >= 0) emit(static_cast<uint32_t>(t[u]), load_one(rowp, t[u]));
            }
        }
        __syncthreads();
        n_chunk = sh.u32[6];
    }

    // 6. Publish: every wave waits for its stores, then one ticket per
    //    workgroup; the last workgroup of the row merges.
    if (tid == 0) store_shared(&a.chunk_count[row * kMaxChunks + chunk], n_chunk);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        const uint32_t ticket =
            __hip_atomic_fetch_add(&a.tickets[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sh.u32[0] = ticket == static_cast<uint32_t>(a.cpr - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (sh.u32[0] == 0u) return;
    merge_row<T>(a, sh, row, p, greedy, k, rowp, hist, H, pen, CHUNK);
}

template <typename T, int EPT>
hipError_t launch_t(const DevArgs& a, hipStream_t s, int gpt) {
    const dim3 grid(static_cast<unsigned>(a.rows * a.cpr));
    const dim3 block(kBlock);
    switch (gpt) {
        case 1: hipLaunchKernelGGL((select_kernel<T, EPT, 1>), grid, block, 0, s, a); break;
        case 4: hipLaunchKernelGGL((select_kernel<T, EPT, 4>), grid, block, 0, s, a); break;
        default: hipLaunchKernelGGL((select_kernel<T, EPT, 16>), grid, block, 0, s, a); break;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_select(const DevArgs& a, hipStream_t stream, int ept, int gpt) {
    if (a.dtype == GE_DTYPE_BF16)
        return ept == 16 ? launch_t<uint16_t, 16>(a, stream, gpt) : launch_t<uint16_t, 64>(a, stream, gpt);
    return ept == 16 ? launch_t<float, 16>(a, stream, gpt) : launch_t<float, 64>(a, stream, gpt);
}

}  // namespace ge
