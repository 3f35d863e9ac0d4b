// gfx950 selection-path kernel of the GemmaEdge token sampler (rows whose
// effective top-k is at most kMaxTopK, and greedy rows).
//
// One launch samples `rows` rows. Each row is split into `cpr` chunks of
// kBlock * EPT logits, one workgroup per chunk. Every workgroup publishes the
// EXACT top-m of its chunk by the sampler's total order (final value
// descending, index ascending), sorted, together with a guarantee G: every
// element of the chunk whose composite key is >= G is in the list. m is a
// speculative count, about k / cpr plus five standard deviations of a
// binomial spread, so the lists are short (k = 40 over 16 chunks: m = 17).
//
// Per chunk:
//   1. issue the chunk's 16-byte loads (consecutive threads on consecutive
//      addresses); while they are in flight, mark the row's unique history
//      ids that fall in the chunk in an LDS bitmap (penalised slots);
//   2. from the maxima of groups of raw logits (penalised slots left out)
//      derive tau, a raw order key with at least m non-penalised logits of
//      the chunk at or above it, and lower tau to the first raw key whose
//      softcapped value equals softcap(tau) (softcap is monotone, so every
//      logit that can tie with tau after capping stays);
//   3. stage the candidates (raw >= that floor, and penalised tokens that can
//      still reach it) in LDS, evaluate their final values there (softcap,
//      then the penalty once per token) and keep the top m, sorted by rank.
//      If the candidates overflow LDS (massive ties) the exact m-th raw key
//      is found by radix select and ties are broken by taking the lowest
//      indices of the boundary class in index order;
//   4. write [G, list] to the row's slot, wait for the stores, take a ticket.
// The last workgroup of the row merges: with Gmax the largest guarantee,
// every element whose composite key is >= Gmax is in some list, so if at
// least k listed entries are >= Gmax they contain the row's top-k. Otherwise
// (a chunk held more than m of the row's top-k) the chunks whose guarantee is
// above the k-th largest listed entry are rescanned with m = k. The merge then
// runs the reference's softmax / min-p / top-p / draw in its exact operation
// order (src/generation.cpp:89-126).
//
// Cross-workgroup data is written with agent-scope relaxed atomic stores: on
// gfx950 these carry the sc1 bit and are coherent across the XCDs' L2s. Each
// wave waits for its stores (s_waitcnt) before the barrier that precedes the
// ticket; no __threadfence() (which writes back and invalidates the XCD's
// whole L2). The merging workgroup reads the lists with agent-scope loads.
//
// No MFMA: nothing here is a contraction. The bound is HBM bandwidth.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <climits>
#include <cstddef>
#include <type_traits>

#include "ge_math.h"
#include "sampler_internal.h"
#include "tie_class.h"
#include "wave_ops.h"

#pragma clang fp contract(off)

namespace ge {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kStage = 2048;    // LDS staging entries (candidates, union)
constexpr int kLoadBatch = 8;   // independent global loads in flight per thread
constexpr uint32_t kPenTag = 0x80000000u;     // staged entry: penalised token

template <typename U>
__device__ __forceinline__ void store_shared(U* p, U v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename U>
__device__ __forceinline__ U load_shared(const U* p) {
    return __hip_atomic_load(const_cast<U*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) { return wave::incl_add(v); }
__device__ __forceinline__ uint32_t wave_max(uint32_t v) { return wave::max_u32(v); }
__device__ __forceinline__ uint32_t wave_min(uint32_t v) { return wave::min_u32(v); }
__device__ __forceinline__ int wave_min_i(int v) { return wave::min_i32(v); }
__device__ __forceinline__ double wave_sum(double v) { return wave::sum_f64(v); }
__device__ __forceinline__ double wave_incl_f64(double v) { return wave::incl_f64(v); }

__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
}

// Chunk list entries carry raw (pre-softcap) values:
//   (raw order key << 32) | (penalised ? 0 : 2^31) | (2^31 - 1 - index).
// Entries are distinct and non-zero; a larger entry has a larger raw value,
// or the same raw value and (unpenalised before penalised, then) a lower
// index. Final values are computed from them by the merging workgroup.
__device__ __forceinline__ uint64_t raw_entry(uint32_t key, uint32_t index, bool pen) {
    return (static_cast<uint64_t>(key) << 32) | ((pen ? 0u : 0x80000000u) | (0x7fffffffu - index));
}
__device__ __forceinline__ uint32_t raw_entry_index(uint64_t e) {
    return 0x7fffffffu - (static_cast<uint32_t>(e) & 0x7fffffffu);
}
__device__ __forceinline__ bool raw_entry_pen(uint64_t e) { return (static_cast<uint32_t>(e) & 0x80000000u) == 0u; }
__device__ __forceinline__ uint32_t raw_entry_low(uint32_t index, bool pen) {
    return (pen ? 0u : 0x80000000u) | (0x7fffffffu - index);
}
// A chunk whose candidates could not be staged publishes this guarantee; the
// merge rescans it exactly.
constexpr uint64_t kGuaranteeFailed = ~0ull;

__device__ __forceinline__ float readlane_f(float v, int i) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
}

__device__ __forceinline__ double readlane_d(double v, int i) {
    const uint64_t b = d2u(v);
    const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(b), i);
    const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(b >> 32), i);
    return u2d((static_cast<uint64_t>(hi) << 32) | lo);
}

// Orders this wave's LDS accesses: LDS operations of one wave execute in
// issue order, so a compiler-level barrier suffices.
// Lane j of the result is v, every other lane keeps old: one v_cndmask with
// the constant lane mask in an SGPR pair, instead of a compare against the
// lane id that writes VCC and the wait states before the select reads it.
template <int j>
__device__ __forceinline__ float put_lane(float old, float v) {
    static_assert(j >= 0 && j < 64, "lane");
    float r;
    asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(old), "v"(v), "s"(1ull << j));
    return r;
}

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Calls f(std::integral_constant<int, J>) for J = 0 .. N-1, in order.
template <int J, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (J < N) {
        f(std::integral_constant<int, J>{});
        static_for<J + 1, N>(f);
    }
}

// threadIdx.x through a volatile move: values derived from it cannot be
// hoisted out of an enclosing loop (the merge's rescans run the chunk routine
// in a loop; hoisted per-thread addresses would stay live across all of it).
__device__ __forceinline__ int opaque_tid() {
    int t;
    asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"(static_cast<int>(threadIdx.x)));
    return t;
}

__device__ __forceinline__ float load_one(const float* rowp, int i) { return rowp[i]; }
__device__ __forceinline__ float load_one(const uint16_t* rowp, int i) { return bf16_to_f32(rowp[i]); }

// Exponent of the lowest set bit of a positive finite float.
__device__ __forceinline__ int lsb_exponent(float e) {
    const uint32_t b = f2u(e);
    const uint32_t ex = b >> 23;
    const uint32_t man = b & 0x7fffffu;
    // Subnormals (ex == 0) count as exponent 1 without the implicit bit:
    // selects, no branch.
    const uint32_t m = ex ? (man | 0x800000u) : man;
    return static_cast<int>(ex ? ex : 1u) - 150 + __builtin_ctz(m);
}

// Largest list a chunk publishes (the top-m by raw value; m may exceed k by
// a few entries so that the merge can certify the k-th).
constexpr int kListCap = kMaxTopK + 8;

// List length each chunk publishes for a row with effective top-k `k`: the
// mean share k / cpr plus four binomial standard deviations plus 4, at least
// 2 and at most k + 4 (the merge certifies its k-th entry against the
// largest m-th entry, so a chunk lists a few more than it contributes), capped
// by the chunk length and the chunk's slot (kSlotWords / cpr words:
// guarantee, count, entries). Every workgroup of the row computes the same m.
// mu = k / cpr with the hardware reciprocal, and its hardware square root:
// any m is correct (it only sizes the lists), and these few instructions are
// deterministic, so every workgroup of a row gets the same m.
__device__ __forceinline__ float spec_mu(uint32_t k, int cpr) {
    return static_cast<float>(k) * __builtin_amdgcn_rcpf(static_cast<float>(cpr));
}
__device__ __forceinline__ uint32_t spec_m(uint32_t k, int cpr, int chunk_len) {
    const float mu = spec_mu(k, cpr);
    uint32_t m = static_cast<uint32_t>(ceilf(mu + 4.0f * __builtin_amdgcn_sqrtf(mu))) + 4u;
    m = min(m, k + 4u);
    m = max(m, 2u);
    m = min(m, static_cast<uint32_t>(kListCap));
    m = min(m, static_cast<uint32_t>(chunk_len));
    m = min(m, static_cast<uint32_t>(kSlotWords / cpr - 2));
    return max(m, 1u);
}

// The merge's first level: it first trusts only the top j1 entries of each
// chunk list (about the mean share plus three standard deviations, plus 2),
// which certifies the row's top k in about 99% of rows with far fewer
// entries to rank; the full lists (level m) are its second try.
__device__ __forceinline__ uint32_t spec_level1(uint32_t k, int cpr, uint32_t m) {
    const float mu = spec_mu(k, cpr);
    const uint32_t j = static_cast<uint32_t>(ceilf(mu + 3.0f * __builtin_amdgcn_sqrtf(mu))) + 2u;
    return min(j, m);
}

struct __align__(16) SelShared {
    uint64_t stage[kStage];      // candidates (staging) / union / sort area; floats of the softmax
    uint64_t list[kListCap];     // chunk routine output: its top-m, sorted descending
    uint64_t top[kMaxTopK];      // merge: the row's top-k, sorted descending
    uint64_t gam[kMaxChunks];    // merge: guarantee of each chunk
    uint64_t exp_tab[32];        // merge: the expf table (2^(i/32)), staged from constant memory
    uint32_t hist[256];
    uint64_t u64[4];
    double f64[kBlock / 64];
    int i32[kBlock / 64];
    uint32_t u32[32];
    uint32_t cnt[kMaxChunks];    // merge: entries each chunk published
};

// Exclusive prefix over the workgroup of one value per thread; also returns
// the total. Uses sh.u32[24..27]; contains barriers (block-uniform).
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t& total, SelShared& sh) {
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

// Sum over the workgroup; block-uniform result. Uses sh.u32[24..27].
__device__ __forceinline__ uint32_t block_sum(uint32_t v, SelShared& sh) {
    uint32_t total;
    (void)block_excl_scan(v, total, sh);
    return total;
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
    const uint32_t total = wave::readlane(incl, 63);
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
// of lo and hi; the second is skipped when at most keep_max keys lie at or
// above the first pass's bin. Returns 0 if fewer than k keys lie in [lo, hi].
// Uses sh.hist and sh.u32[20..22]; block-uniform.
template <typename Visit>
__device__ __forceinline__ uint32_t block_kth(uint32_t lo, uint32_t hi, uint32_t k, Visit&& visit,
                                              SelShared& sh, uint32_t keep_max = 0u) {
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
    const uint32_t in_bin = short_set ? 0u : sh.hist[d1];
    __syncthreads();
    if (short_set) return 0u;
    const uint32_t pre = base1 + d1;
    if (shift1 == 0) return pre;
    if (above + in_bin <= keep_max) return pre << shift1;  // few enough at or above its bin
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

// hist[bin] += 1 for every active lane with `in`; when all of them share the
// first one's bin (equal or sorted keys: -inf-masked rows, long runs), one
// atomic adds the count instead of 64 to one address, which LDS serialises.
__device__ __forceinline__ void hist_add_wave(uint32_t* hist, bool in, uint32_t bin) {
    const uint64_t act = __ballot(in);
    if (act == 0ull) return;
    const int first = __ffsll(static_cast<unsigned long long>(act)) - 1;
    const uint32_t b0 = wave::readlane(bin, first);
    if (__ballot(in && bin == b0) == act) {
        if (__lane_id() == first) atomicAdd(&hist[b0], static_cast<uint32_t>(__popcll(act)));
    } else if (in) {
        atomicAdd(&hist[bin], 1u);
    }
}

// The exact k-th largest of the keys (>= 1) that `visit` presents: 8-bit
// radix digits from the highest bit where lo and hi differ, narrowed until
// every bit is fixed. Returns 0 if fewer than k keys lie in [lo, hi].
// Block-uniform; uses sh.hist and sh.u32[20..22]. `visit` may call its
// function from divergent code: the counts are wave-aggregated over the
// lanes that are active.
template <typename Visit>
__device__ __forceinline__ uint32_t block_kth_exact(uint32_t lo, uint32_t hi, uint32_t k, Visit&& visit, SelShared& sh) {
    const int tid = threadIdx.x;
    if (lo > hi || k == 0) return 0u;
    const uint32_t diff = lo ^ hi;
    int hb = diff ? 31 - __clz(static_cast<int>(diff)) : 0;
    int shift = max(hb - 7, 0);
    int width = hb - shift + 1;
    uint32_t fixed = (hb + 1 >= 32) ? 0u : ~((1u << (hb + 1)) - 1u);
    uint32_t prefix = lo & fixed;
    uint32_t need = k;
    for (;;) {
        for (int i = tid; i < 256; i += kBlock) sh.hist[i] = 0u;
        __syncthreads();
        const uint32_t dmask = (1u << width) - 1u;
        visit([&](uint32_t key) {
            hist_add_wave(sh.hist, key >= lo && key <= hi && (key & fixed) == prefix, (key >> shift) & dmask);
        });
        __syncthreads();
        if (tid < 64) find_bin_desc(sh.hist, need, &sh.u32[20]);
        __syncthreads();
        const uint32_t d = sh.u32[20];
        const uint32_t above = sh.u32[21];
        const bool short_set = sh.u32[22] != 0u;
        __syncthreads();
        if (short_set) return 0u;
        need -= above;
        prefix |= d << shift;
        fixed |= dmask << shift;
        if (shift == 0) return prefix;
        const int ns = max(shift - 8, 0);
        width = shift - ns;
        shift = ns;
    }
}

// Descending bitonic sort of s[0, n), n a power of two <= kStage, by the
// whole workgroup through LDS. In each stage a thread's pairs are disjoint, so
// it loads all of them before comparing and storing any: one LDS round trip
// per stage instead of one per pair (the compiler cannot prove that a pair's
// stores miss the next pair's loads).
__device__ __forceinline__ void bitonic_desc_block(uint64_t* s, uint32_t n) {
    constexpr int kPairs = kStage / 2 / kBlock;  // pairs per thread at most
    const int tid = threadIdx.x;
    for (uint32_t size = 2; size <= n; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            uint64_t x[kPairs], y[kPairs];
#pragma unroll
            for (int u = 0; u < kPairs; ++u) {
                const uint32_t i = static_cast<uint32_t>(u * kBlock + tid);
                const uint32_t pos = 2 * i - (i & (stride - 1));
                if (i < n / 2) {
                    x[u] = s[pos];
                    y[u] = s[pos + stride];
                }
            }
#pragma unroll
            for (int u = 0; u < kPairs; ++u) {
                const uint32_t i = static_cast<uint32_t>(u * kBlock + tid);
                const uint32_t pos = 2 * i - (i & (stride - 1));
                const bool desc = (pos & size) == 0;
                if (i < n / 2 && (x[u] < y[u]) == desc) {
                    s[pos] = y[u];
                    s[pos + stride] = x[u];
                }
            }
            __syncthreads();
        }
    }
}

// dst[0, min(n, m)) = the largest min(n, m) of the distinct non-zero keys
// src[0, n), sorted descending. src is clobbered. n <= kStage. Block-uniform.
__device__ __forceinline__ uint32_t select_top(uint64_t* src, uint32_t n, uint32_t m, uint64_t* dst) {
    const int tid = threadIdx.x;
    const uint32_t out = min(n, m);
    if (n <= static_cast<uint32_t>(kBlock)) {
        // Rank by counting: every key is distinct, so its rank is the number
        // of larger keys. Two keys per 16-byte LDS read (src[n] padded).
        if (tid == 0 && (n & 1u)) src[n] = 0ull;
        __syncthreads();
        if (static_cast<uint32_t>(tid) < n) {
            const uint64_t x = src[tid];
            uint32_t r = 0;
            const ulonglong2* p2 = reinterpret_cast<const ulonglong2*>(src);
#pragma unroll 8
            for (uint32_t j = 0; j < (n + 1) / 2; ++j) {
                const ulonglong2 q = p2[j];
                r += q.x > x ? 1u : 0u;
                r += q.y > x ? 1u : 0u;
            }
            if (r < m) dst[r] = x;
        }
        __syncthreads();
        return out;
    }
    uint32_t n2 = 1;
    while (n2 < n) n2 <<= 1;
    for (uint32_t i = n + tid; i < n2; i += kBlock) src[i] = 0ull;
    __syncthreads();
    bitonic_desc_block(src, n2);
    for (uint32_t i = tid; i < out; i += kBlock) dst[i] = src[i];
    __syncthreads();
    return out;
}

// r + the number of the four keys a, b, c, d greater than x. Each compare
// writes its own SGPR pair and feeds an add-with-carry, and every mask is
// read three instructions after it is written: no compare into VCC followed
// by wait states and a select, as the compiler emits for (q > x ? 1 : 0).
__device__ __forceinline__ uint32_t add_greater4(uint32_t r, uint64_t a, uint64_t b, uint64_t c, uint64_t d,
                                                 uint64_t x) {
    uint64_t s0, s1, s2, s3, co;
    asm("v_cmp_gt_u64_e64 %1, %6, %10\n\t"
        "v_cmp_gt_u64_e64 %2, %7, %10\n\t"
        "v_cmp_gt_u64_e64 %3, %8, %10\n\t"
        "v_cmp_gt_u64_e64 %4, %9, %10\n\t"
        "v_addc_co_u32_e64 %0, %5, %0, 0, %1\n\t"
        "v_addc_co_u32_e64 %0, %5, %0, 0, %2\n\t"
        "v_addc_co_u32_e64 %0, %5, %0, 0, %3\n\t"
        "v_addc_co_u32_e64 %0, %5, %0, 0, %4"
        : "+v"(r), "=&s"(s0), "=&s"(s1), "=&s"(s2), "=&s"(s3), "=&s"(co)
        : "v"(a), "v"(b), "v"(c), "v"(d), "v"(x));
    return r;
}

// dst[0, min(n, m)) = the largest min(n, m) of the distinct non-zero keys
// src[0, n) (n <= kBlock), sorted descending, by counting with exact 64-bit
// compares on keys read in pairs from LDS broadcasts. The caller has padded
// src[n, roundup(n, 8)) with zeros and synchronised. Block-uniform (one
// barrier at the end).
__device__ __forceinline__ uint32_t rank_top_exact(const uint64_t* src, uint32_t n, uint32_t m, uint64_t* dst) {
    const int tid = threadIdx.x;
    if (static_cast<uint32_t>(tid) < n) {
        const uint64_t x = src[tid];
        const ulonglong2* p2 = reinterpret_cast<const ulonglong2*>(src);
        uint32_t r = 0;
        for (uint32_t j = 0; j < (n + 7u) / 8u; ++j) {
            const ulonglong2 q0 = p2[4 * j + 0], q1 = p2[4 * j + 1], q2 = p2[4 * j + 2], q3 = p2[4 * j + 3];
            r = add_greater4(r, q0.x, q0.y, q1.x, q1.y, x);
            r = add_greater4(r, q2.x, q2.y, q3.x, q3.y, x);
        }
        if (r < m) dst[r] = x;
    }
    __syncthreads();
    return min(n, m);
}

// The row-level context every workgroup of a row shares.
struct RowCtx {
    const void* rowp;   // the row's logits
    const int32_t* hist;
    int row;
    int V;
    int H;
    int vec_ok;         // rows are 16-byte aligned
    bool pen;           // the penalty applies (history non-empty, r != 1)
    float r;
    float cap;
};

// Slot layout extension of the lean rows (see merge_lean): the list's final
// keys at words [fin, fin + L) and the capped value key of the j1-th entry
// at word `bound`, next to [guarantee, count, raw entries (at most L)].
struct LeanList {
    bool on;
    uint32_t j1;     // merge level 1
    uint32_t cap;    // L: entries a lean list may hold
    uint32_t fin;    // word of the first final key
    uint32_t bound;  // word of the capped j1-th entry
    // Final-order lists (merge_fs, k above 64): the chunk publishes its top m
    // by raw order as final composite keys sorted by final value, with the
    // capped values of its m-th (word 0) and j1-th (last word of the slot)
    // raw entries as bounds. The chunk's list then comes from LDS, not from
    // the one-wave direct rank.
    bool fs;
};

// Batches of the rescans' loads: SBE elements per thread (whole groups of W;
// a template argument of the routines below, 0 for one group) are requested
// before any is used. Loads at clamped addresses and unconditional: a load
// under a lane mask is followed by a wait for every load in flight, which
// made every element's load a round trip of its own. Larger batches hold
// more registers: the single-pass kernel's rescans use 16 elements, the
// select kernel's (already at its register limit) one group.
constexpr int kSlowBatchStream = 8;

// Groups v0 .. v0 + SB - 1 of this thread (group v: elements e0 .. e0 + W - 1,
// e0 = c0 + (v * kBlock + tid) * W); elements at or past cend read as NaN.
template <typename T, int W, int SB>
__device__ __forceinline__ void load_groups(const T* rowp, int c0, int cend, int tid, int v0, float (&x)[SB][W]) {
    if (c0 + (v0 + SB) * kBlock * W <= cend) {  // the whole batch in range (block-uniform)
#pragma unroll
        for (int b = 0; b < SB; ++b) {
            const int e0 = c0 + ((v0 + b) * kBlock + tid) * W;
#pragma unroll
            for (int j = 0; j < W; ++j) x[b][j] = load_one(rowp, e0 + j);
        }
    } else {
#pragma unroll
        for (int b = 0; b < SB; ++b) {
            const int e0 = c0 + ((v0 + b) * kBlock + tid) * W;
#pragma unroll
            for (int j = 0; j < W; ++j) {
                const float t = load_one(rowp, min(e0 + j, cend - 1));
                x[b][j] = e0 + j < cend ? t : NAN;
            }
        }
    }
}

// Builds the chunk's penalty bitmap in pbits (one bit per element of
// [c0, c0 + CHUNK)) from the row's history. Block-uniform (barriers).
template <int CHUNK>
__device__ __forceinline__ void build_penalty_bitmap(const RowCtx& rc, int c0, int cend, int tid, uint32_t* pbits) {
    for (int w = tid; w < CHUNK / 32; w += kBlock) pbits[w] = 0u;
    __syncthreads();
    for (int base = 0; base < rc.H; base += kBlock * kLoadBatch) {
        int t[kLoadBatch];
#pragma unroll
        for (int u = 0; u < kLoadBatch; ++u) {
            const int j = base + u * kBlock + tid;
            t[u] = j < rc.H ? rc.hist[j] : -1;
        }
#pragma unroll
        for (int u = 0; u < kLoadBatch; ++u)
            if (t[u] >= c0 && t[u] < cend) atomicOr(&pbits[(t[u] - c0) >> 5], 1u << ((t[u] - c0) & 31));
    }
    __syncthreads();
}

// Exact top-m of one chunk, for the rare cases: candidates that overflow LDS
// in the streaming pass (massive ties, or a bound far below the m-th value)
// and the merge's rescans. Same contract as chunk_topm. It keeps registers
// low: runtime loops over batches of kSlowBatch elements per thread,
// reloading the chunk from memory (L2 / MALL) in every pass.
//   1. R = the exact m-th largest non-penalised raw order key (radix select);
//   2. lo..hi = the raw keys whose softcapped value equals R's (its class);
//   3. candidates: every non-penalised element above the class, the
//      m - (that count) lowest-index members of the class (counted in index
//      order), and every penalised token that can reach the class;
//   4. final values, top m, sorted.
template <typename T, int EPT, int SBE>
__device__ __forceinline__ uint64_t chunk_slow(const RowCtx& rc, int c0, uint32_t m, uint32_t* pbits,
                                               SelShared& sh, uint32_t& n_out, bool& ok) {
    constexpr int W = sizeof(T) == 4 ? 4 : 8;
    constexpr int NV = EPT / W;
    constexpr int CHUNK = kBlock * EPT;
    const int tid = opaque_tid();
    const int lane = __lane_id();
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const T* rowp = static_cast<const T*>(rc.rowp);
    const int cend = min(c0 + CHUNK, rc.V);
    ok = true;
    if (rc.pen) build_penalty_bitmap<CHUNK>(rc, c0, cend, tid, pbits);
    auto is_pen = [&](int e) -> bool {
        return rc.pen && ((pbits[(e - c0) >> 5] >> ((e - c0) & 31)) & 1u);
    };
    constexpr int SB = SBE / W < 1 ? 1 : (SBE / W < NV ? SBE / W : NV);  // groups per batch
    static_assert(NV % SB == 0, "batches of whole groups");
    auto visit_np = [&](auto&& f) {
#pragma unroll 1
        for (int v0 = 0; v0 < NV; v0 += SB) {
            float x[SB][W];
            load_groups<T, W, SB>(rowp, c0, cend, tid, v0, x);
#pragma unroll
            for (int b = 0; b < SB; ++b) {
                const int e0 = c0 + ((v0 + b) * kBlock + tid) * W;
#pragma unroll
                for (int j = 0; j < W; ++j)
                    if (e0 + j < cend && !is_pen(e0 + j)) f(order_key(x[b][j]));
            }
        }
    };
    const uint32_t R = block_kth_exact(1u, 0xffffffffu, m, visit_np, sh);
    uint32_t lo = 0u, hi = 0xffffffffu;  // R == 0: fewer than m, take them all
    if (R != 0u) {
        if (wave == 0) {
            const uint32_t l = tie_floor(R, rc.cap);
            const uint32_t h = tie_ceil(R, rc.cap);
            if (lane == 0) {
                sh.u32[4] = l;
                sh.u32[5] = h;
            }
        }
        __syncthreads();
        lo = sh.u32[4];
        hi = sh.u32[5];
    }
    uint32_t above = 0;
    if (R != 0u) {
        visit_np([&](uint32_t key) { above += key > hi ? 1u : 0u; });
        above = block_sum(above, sh);
    }
    const uint32_t q = R != 0u ? m - above : 0xffffffffu;  // class members to take
    // Penalised tokens leave the raw order (a penalty below 1 can even lift
    // one above every bound taken from raw values), so the penalised
    // candidates are the top m penalised tokens by final value (ties at the
    // m-th taken in index order): the chunk's top m lies in the union of
    // that set and the unpenalised candidates above, at most 2m <= kStage
    // entries, so this routine always completes.
    auto pen_key = [&](float x) { return order_key(penalize(softcap(x, rc.cap), rc.r)); };
    uint32_t pk = 0u;             // m-th largest penalised final key (0: fewer than m, all)
    uint32_t pq = 0xffffffffu;    // penalised tokens of key pk to take
    if (rc.pen) {
        auto visit_pen = [&](auto&& f) {
#pragma unroll 1
            for (int v0 = 0; v0 < NV; v0 += SB) {
                float x[SB][W];
                load_groups<T, W, SB>(rowp, c0, cend, tid, v0, x);
#pragma unroll
                for (int b = 0; b < SB; ++b) {
                    const int e0 = c0 + ((v0 + b) * kBlock + tid) * W;
#pragma unroll
                    for (int j = 0; j < W; ++j)
                        if (e0 + j < cend && is_pen(e0 + j)) f(pen_key(x[b][j]));
                }
            }
        };
        pk = block_kth_exact(1u, 0xffffffffu, m, visit_pen, sh);
        if (pk != 0u) {
            uint32_t pabove = 0;
            visit_pen([&](uint32_t key) { pabove += key > pk ? 1u : 0u; });
            pq = m - block_sum(pabove, sh);
        }
    }
    // Stage in index order: per group, the class ranks and the candidates'
    // positions are exclusive scans over the threads.
    uint32_t cls_before = 0, pcls_before = 0, n_c = 0;
#pragma unroll 1
    for (int v0 = 0; v0 < NV; v0 += SB) {
        float xb[SB][W];
        load_groups<T, W, SB>(rowp, c0, cend, tid, v0, xb);
#pragma unroll
        for (int b = 0; b < SB; ++b) {
            const float (&x)[W] = xb[b];
            const int e0 = c0 + ((v0 + b) * kBlock + tid) * W;
            uint32_t cls = 0, pen = 0, valid = 0;
#pragma unroll
            for (int j = 0; j < W; ++j) {
                const uint32_t key = order_key(x[j]);
                const bool in = e0 + j < cend;
                const bool pj = in && is_pen(e0 + j);
                valid |= static_cast<uint32_t>(in) << j;
                pen |= static_cast<uint32_t>(pj) << j;
                cls |= static_cast<uint32_t>(in && !pj && key >= lo && key <= hi) << j;
            }
            uint32_t cls_total;
            const uint32_t cbase = cls_before + block_excl_scan(static_cast<uint32_t>(__popc(cls)), cls_total, sh);
            cls_before += cls_total;
            uint32_t pcls = 0, pbig = 0;  // penalised: final key == pk / > pk
            if (pen != 0u && pk != 0u) {
#pragma unroll
                for (int j = 0; j < W; ++j) {
                    if (!((pen >> j) & 1u)) continue;
                    const uint32_t fk = pen_key(x[j]);
                    pcls |= static_cast<uint32_t>(fk == pk) << j;
                    pbig |= static_cast<uint32_t>(fk > pk) << j;
                }
            }
            uint32_t pbase = 0;
            if (pk != 0u) {
                uint32_t pcls_total;
                pbase = pcls_before + block_excl_scan(static_cast<uint32_t>(__popc(pcls)), pcls_total, sh);
                pcls_before += pcls_total;
            }
            uint32_t cand = 0;
#pragma unroll
            for (int j = 0; j < W; ++j) {
                const uint32_t key = order_key(x[j]);
                bool c;
                if ((pen >> j) & 1u) {
                    c = pk == 0u || ((pbig >> j) & 1u) ||
                        (((pcls >> j) & 1u) && pbase + static_cast<uint32_t>(__popc(pcls & ((1u << j) - 1u))) < pq);
                } else if ((cls >> j) & 1u) {
                    c = cbase + static_cast<uint32_t>(__popc(cls & ((1u << j) - 1u))) < q;
                } else {
                    c = ((valid >> j) & 1u) && key > hi;
                }
                cand |= static_cast<uint32_t>(c) << j;
            }
            uint32_t cand_total;
            const uint32_t pos = n_c + block_excl_scan(static_cast<uint32_t>(__popc(cand)), cand_total, sh);
            if (n_c + cand_total > static_cast<uint32_t>(kStage)) {
                ok = false;
                n_out = 0;
                return ~0ull;
            }
            uint32_t o = pos;
#pragma unroll
            for (int j = 0; j < W; ++j) {
                if ((cand >> j) & 1u) {
                    const uint32_t tag = static_cast<uint32_t>(e0 + j) | (((pen >> j) & 1u) ? kPenTag : 0u);
                    sh.stage[o++] = (static_cast<uint64_t>(tag) << 32) | f2u(x[j]);
                }
            }
            n_c += cand_total;
        }
    }
    __syncthreads();
    for (uint32_t i = tid; i < n_c; i += kBlock) {
        const uint64_t x = sh.stage[i];
        const uint32_t tag = static_cast<uint32_t>(x >> 32);
        float f = softcap(u2f(static_cast<uint32_t>(x)), rc.cap);
        if (tag & kPenTag) f = penalize(f, rc.r);
        sh.stage[i] = composite(order_key(f), tag & ~kPenTag);
    }
    __syncthreads();
    n_out = select_top(sh.stage, n_c, m, sh.list);
    // Every element left out is below the m-th listed key (or the chunk
    // listed everything).
    return n_out == m ? sh.list[m - 1] : 0ull;
}

// With a penalty below 1 a penalised token can rise above any bound taken
// from raw values, so every penalised candidate of the chunk is listed: those
// among sh.stage[0, n_c) below the m-th entry `last` are written to the
// chunk's slot after the top m (slot[2 + m ...], stride words in all).
// Returns the number appended; ok = false if they do not fit. Block-uniform.
__device__ __forceinline__ uint32_t append_penalised(SelShared& sh, uint32_t n_c, uint32_t m, uint64_t last,
                                                     uint64_t* slot, uint32_t stride, bool& ok) {
    const int tid = threadIdx.x;
    if (tid == 0) sh.u32[17] = 0u;
    __syncthreads();
    for (uint32_t i = tid; i < n_c; i += kBlock) {
        const uint64_t x = sh.stage[i];
        if (x != 0ull && raw_entry_pen(x) && x < last) {
            const uint32_t pos = atomicAdd(&sh.u32[17], 1u);
            if (m + 2u + pos < stride) store_shared(&slot[m + 2u + pos], x);
        }
    }
    __syncthreads();
    const uint32_t extra = sh.u32[17];
    __syncthreads();
    if (m + 2u + extra > stride) ok = false;
    return extra;
}

// Exact raw top-m of one chunk for the rare cases of the streaming pass
// (candidates that overflow LDS: massive ties, NaN-heavy or partial chunks).
// Same contract as chunk_topm; the penalty bitmap pbits is already built.
// Runtime loops over batches of kSlowBatch elements per thread, reloading the
// chunk from memory (L2 / MALL) in every pass:
//   1. R = the exact m-th largest raw order key (radix select);
//   2. Lq = the (m - #above R)-th largest entry low word among the keys
//      equal to R (low words are distinct), so that exactly m entries are
//      >= raw_entry(R, Lq);
//   3. stage those (and, with a penalty below 1, every penalised element),
//      sort, keep the top m.
template <typename T, int EPT, int SBE>
__device__ __forceinline__ uint64_t chunk_slow_raw(const RowCtx& rc, int c0, uint32_t m, const uint32_t* pbits,
                                                   SelShared& sh, uint64_t* slot, uint32_t stride,
                                                   uint32_t& n_top, uint32_t& n_out, bool& ok) {
    constexpr int W = sizeof(T) == 4 ? 4 : 8;
    constexpr int NV = EPT / W;
    constexpr int CHUNK = kBlock * EPT;
    const int tid = opaque_tid();
    const T* rowp = static_cast<const T*>(rc.rowp);
    const int cend = min(c0 + CHUNK, rc.V);
    const bool pen_all = rc.pen && !(rc.r >= 1.0f);
    ok = true;
    auto is_pen = [&](int e) -> bool {
        return rc.pen && ((pbits[(e - c0) >> 5] >> ((e - c0) & 31)) & 1u);
    };
    constexpr int SB = SBE / W < 1 ? 1 : (SBE / W < NV ? SBE / W : NV);  // groups per batch
    static_assert(NV % SB == 0, "batches of whole groups");
    auto visit_keys = [&](auto&& f) {
#pragma unroll 1
        for (int v0 = 0; v0 < NV; v0 += SB) {
            float x[SB][W];
            load_groups<T, W, SB>(rowp, c0, cend, tid, v0, x);
#pragma unroll
            for (int b = 0; b < SB; ++b) {
                const int e0 = c0 + ((v0 + b) * kBlock + tid) * W;
#pragma unroll
                for (int j = 0; j < W; ++j)
                    if (e0 + j < cend) f(order_key(x[b][j]));
            }
        }
    };
    const uint32_t R = block_kth_exact(1u, 0xffffffffu, m, visit_keys, sh);
    uint32_t lq = 0u;  // R == 0: fewer than m elements, list them all
    if (R != 0u) {
        uint32_t above = 0;
        visit_keys([&](uint32_t key) { above += key > R ? 1u : 0u; });
        above = block_sum(above, sh);
        const uint32_t q = m - above;  // >= 1
        auto visit_lows = [&](auto&& f) {
#pragma unroll 1
            for (int v0 = 0; v0 < NV; v0 += SB) {
                float x[SB][W];
                load_groups<T, W, SB>(rowp, c0, cend, tid, v0, x);
#pragma unroll
                for (int b = 0; b < SB; ++b) {
                    const int e0 = c0 + ((v0 + b) * kBlock + tid) * W;
#pragma unroll
                    for (int j = 0; j < W; ++j)
                        if (e0 + j < cend && order_key(x[b][j]) == R)
                            f(raw_entry_low(static_cast<uint32_t>(e0 + j), is_pen(e0 + j)));
                }
            }
        };
        lq = block_kth_exact(1u, 0xffffffffu, q, visit_lows, sh);
    }
    const uint64_t thr = R != 0u ? ((static_cast<uint64_t>(R) << 32) | lq) : 0ull;
    uint32_t n_c = 0;
#pragma unroll 1
    for (int v0 = 0; v0 < NV; v0 += SB) {
        float xb[SB][W];
        load_groups<T, W, SB>(rowp, c0, cend, tid, v0, xb);
#pragma unroll
        for (int b = 0; b < SB; ++b) {
            const float (&x)[W] = xb[b];
            const int e0 = c0 + ((v0 + b) * kBlock + tid) * W;
            uint64_t ent[W];
            uint32_t cand = 0;
#pragma unroll
            for (int j = 0; j < W; ++j) {
                const bool in = e0 + j < cend;
                const bool pj = in && is_pen(e0 + j);
                ent[j] = raw_entry(order_key(x[j]), static_cast<uint32_t>(e0 + j), pj);
                cand |= static_cast<uint32_t>(in && (ent[j] >= thr || (pen_all && pj))) << j;
            }
            uint32_t total;
            uint32_t pos = n_c + block_excl_scan(static_cast<uint32_t>(__popc(cand)), total, sh);
            if (n_c + total > static_cast<uint32_t>(kStage)) {
                ok = false;
                n_top = n_out = 0;
                return kGuaranteeFailed;
            }
#pragma unroll
            for (int j = 0; j < W; ++j)
                if ((cand >> j) & 1u) sh.stage[pos++] = ent[j];
            n_c += total;
        }
    }
    __syncthreads();
    n_top = select_top(sh.stage, n_c, m, sh.list);
    n_out = n_top;
    const uint64_t g = (R != 0u && n_top == m) ? sh.list[m - 1] : 0ull;
    if (pen_all && n_c > m) n_out += append_penalised(sh, n_c, m, g, slot, stride, ok);
    return ok ? g : kGuaranteeFailed;
}

// The t-th largest (1 <= t <= 64) of the wave's 64 keys, wave-uniform. For
// small t, t rounds of "maximum, then retire one lane holding it"; else a
// bit-by-bit ballot search.
__device__ __forceinline__ uint32_t wave_kth(uint32_t key, uint32_t t) {
    if (t > 8u) return wave::kth_largest(key, t);
    const int lane = __lane_id();
    uint32_t mx = 0u;
    for (uint32_t i = 0; i < t; ++i) {
        mx = wave::max_u32(key);
        const uint64_t eq = __ballot(key == mx);
        if (lane == __ffsll(static_cast<unsigned long long>(eq)) - 1) key = 0u;
    }
    return mx;
}

// Per-wave staging segments: wave w stages its keys in
// sh.stage[w * kSeg, w * kSeg + cnt[w]), padded with a zero key to an even
// count (the rank reads keys in pairs).
constexpr int kSeg = kStage / (kBlock / 64);
// sh.u32 words holding the segment counts. Not shared with any other helper's
// scratch: block_excl_scan (24..27) can run right after the counts are read.
constexpr int kSegCount = 28;
// Up to this many entries the merge ranks them by counting directly.
constexpr uint32_t kRankDirect = 96;

// dst[0, min(n, m)) = the largest of the n <= kBlock distinct non-zero keys in
// the segments, sorted descending (rank by counting, keys in pairs).
// Block-uniform (one barrier at the end).
__device__ __forceinline__ void seg_rank_top(const uint64_t* stage, const uint32_t (&cnt)[kBlock / 64],
                                             uint32_t n, uint32_t m, uint64_t* dst) {
    const int tid = threadIdx.x;
    if (static_cast<uint32_t>(tid) < n) {
        int w = 0;
        uint32_t i = static_cast<uint32_t>(tid);
        while (i >= cnt[w]) {
            i -= cnt[w];
            ++w;
        }
        const uint64_t x = stage[w * kSeg + i];
        uint32_t rk = 0;
#pragma unroll
        for (int v = 0; v < kBlock / 64; ++v) {
            const ulonglong2* sv = reinterpret_cast<const ulonglong2*>(stage + v * kSeg);
#pragma unroll 4
            for (uint32_t j = 0; j < (cnt[v] + 1) / 2; ++j) {
                const ulonglong2 q = sv[j];
                rk += q.x > x ? 1u : 0u;
                rk += q.y > x ? 1u : 0u;
            }
        }
        if (rk < m) dst[rk] = x;
    }
    __syncthreads();
}

// Moves the n keys of the segments to stage[0, n) (n <= kStage). Block-uniform.
__device__ __forceinline__ void seg_gather(uint64_t* stage, const uint32_t (&cnt)[kBlock / 64], uint32_t n) {
    const int tid = threadIdx.x;
    uint64_t tmp[kStage / kBlock];
#pragma unroll
    for (int q = 0; q < kStage / kBlock; ++q) {
        uint32_t i = static_cast<uint32_t>(q * kBlock + tid);
        tmp[q] = 0ull;
        if (i < n) {
            int w = 0;
            while (i >= cnt[w]) {
                i -= cnt[w];
                ++w;
            }
            tmp[q] = stage[w * kSeg + i];
        }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kStage / kBlock; ++q) {
        const uint32_t i = static_cast<uint32_t>(q * kBlock + tid);
        if (i < n) stage[i] = tmp[q];
    }
    __syncthreads();
}

// Raw top-m of one chunk (elements [c0, min(c0 + CHUNK, V))): the m largest
// raw list entries (raw value descending; see raw_entry), sorted descending
// into sh.list[0, n_top). With a penalty below 1, every penalised element of
// the chunk is listed too (appended to the slot after the top m; n_out counts
// them all). Returns the chunk's guarantee g: every element left out has a
// raw entry < g, so (softcap being monotone and a penalty >= 1 never raising
// a value) its final value is at most softcap(value of g); g = 0 when the
// chunk listed everything, kGuaranteeFailed when its candidates could not be
// staged. The list being sorted, its j-th entry is such a guarantee for the
// first j entries too. No softcap is evaluated here: the merge caps only what
// it needs. Block-uniform; every thread returns the same values.
//
// The bound tau: at least m elements of the chunk have a raw order key >=
// tau (from the maxima of groups of logits). Every element >= tau is staged,
// so the top m of the staged entries is the chunk's top m.
template <typename T, int EPT>
__device__ __forceinline__ uint64_t chunk_topm(const RowCtx& rc, int c0, uint32_t m, uint32_t* pbits,
                                               SelShared& sh, uint64_t* slot, uint32_t stride, const LeanList& ll,
                                               uint32_t& n_top, uint32_t& n_out, bool& direct, bool& ok) {
    constexpr int W = sizeof(T) == 4 ? 4 : 8;  // elements per 16-byte load
    constexpr int NV = EPT / W;                 // 16-byte loads per thread
    constexpr int NW = EPT * sizeof(T) / 4;     // 32-bit words per thread
    constexpr int CHUNK = kBlock * EPT;
    constexpr int NG = EPT / 4;                 // groups of 4 slots per thread
    static_assert(EPT % W == 0 && EPT <= 64 && EPT % 4 == 0, "bad tiling");

    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int wave = tid >> 6;
    const T* rowp = static_cast<const T*>(rc.rowp);
    const int cend = min(c0 + CHUNK, rc.V);
    const bool pen_all = rc.pen && !(rc.r >= 1.0f);
    ok = true;
    direct = false;

    // Slot s of this thread is element c0 + ((s / W) * kBlock + tid) * W + s % W.
    auto elem = [&](int s) { return c0 + ((s / W) * kBlock + tid) * W + (s % W); };
    constexpr uint32_t kHole = 0x7fc00000u;  // NaN placed in out-of-range slots

    // 1. The first kBlock * kLoadBatch history ids, then the chunk's 16-byte
    //    loads; both round trips overlap (loads return in issue order). The
    //    id loads are unconditional (index clamped, validity checked at use)
    //    so that the wait for them counts only them, not the logits.
    int hid[kLoadBatch];
    if (rc.pen) {
#pragma unroll
        for (int u = 0; u < kLoadBatch; ++u) hid[u] = rc.hist[min(u * kBlock + tid, rc.H - 1)];
    }
    // 2. The penalty bitmap (one bit per element of the chunk) from the row's
    //    history. Built on each load path separately: on the vector path
    //    after the logit loads are issued, while they are in flight (the ids
    //    arrive first); a build after the paths join would wait for every
    //    load of either path.
    auto mark_history = [&]() {
        if (!rc.pen) return;
        for (int w = tid; w < CHUNK / 32; w += kBlock) pbits[w] = 0u;
        __syncthreads();
        for (int base = 0; base < rc.H; base += kBlock * kLoadBatch) {
            if (base > 0) {
#pragma unroll
                for (int u = 0; u < kLoadBatch; ++u) hid[u] = rc.hist[min(base + u * kBlock + tid, rc.H - 1)];
            }
#pragma unroll
            for (int u = 0; u < kLoadBatch; ++u)
                if (base + u * kBlock + tid < rc.H && hid[u] >= c0 && hid[u] < cend)
                    atomicOr(&pbits[(hid[u] - c0) >> 5], 1u << ((hid[u] - c0) & 31));
        }
    };
    uint32_t d[NW];
    uint64_t vmask = ~0ull;  // in-range slots
    auto value = [&](int s) -> float {
        if constexpr (W == 4) return u2f(d[s]);
        else return u2f((s % 2 == 0) ? (d[s / 2] << 16) : (d[s / 2] & 0xffff0000u));
    };
    // bf16: makes the packed words opaque so that the unpacked floats of one
    // phase are recomputed in the next instead of being held in registers.
    auto fence_words = [&]() {
        if constexpr (W == 8) {
#pragma unroll
            for (int i = 0; i < NW; ++i) asm volatile("" : "+v"(d[i]));
        }
    };
    if (rc.vec_ok && c0 + CHUNK <= rc.V) {
        // Streaming loads: each logit is read once, so they carry the
        // nontemporal hint and do not displace the lists and history in L2.
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const u32x4 q = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rowp + c0 + (v * kBlock + tid) * W));
            d[4 * v + 0] = q.x;
            d[4 * v + 1] = q.y;
            d[4 * v + 2] = q.z;
            d[4 * v + 3] = q.w;
        }
        if constexpr (EPT < 64) vmask = (1ull << EPT) - 1ull;
        mark_history();
    } else {
        mark_history();
        vmask = 0ull;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int n_in = min(max(cend - (c0 + (v * kBlock + tid) * W), 0), W);
            vmask |= static_cast<uint64_t>((1u << n_in) - 1u) << (v * W);
        }
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

    // 3. The bound. Maxima of groups of 4 raw values (fmaxf ignores the NaN
    //    of out-of-range slots).
    float gm[NG];
    float lmf = NAN;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        float x = value(g * 4);
#pragma unroll
        for (int j = 1; j < 4; ++j) x = fmaxf(x, value(g * 4 + j));
        gm[g] = x;
        lmf = fmaxf(lmf, x);
    }
    fence_words();
    const uint32_t lkey = order_key(lmf);
    uint32_t tau;
    if (m <= 4u * 64u) {
        // Each wave: the ceil(m/4)-th largest of its 64 lane maxima; the
        // smallest of the four leaves >= m elements at or above it (a looser
        // bound than the radix select below over the group maxima for large
        // m, but far cheaper: for m = 100 it cut the bound from about 5.5 us
        // to a ballot search, and the rank absorbs the extra candidates). The
        // barrier also orders the bitmap's marks before the staging reads.
        const uint32_t tw = wave_kth(lkey, (m + 3u) / 4u);
        if (lane == 0) sh.u32[8 + wave] = tw;
        __syncthreads();
        tau = min(min(sh.u32[8], sh.u32[9]), min(sh.u32[10], sh.u32[11]));
    } else {
        uint32_t gmn = 0xffffffffu;
#pragma unroll
        for (int g = 0; g < NG; ++g) gmn = min(gmn, order_key(gm[g]));
        const uint32_t gmx = wave_max(lkey);
        gmn = wave_min(gmn);
        if (lane == 0) {
            sh.u32[8 + wave] = gmx;
            sh.u32[12 + wave] = gmn;
        }
        __syncthreads();
        const uint32_t bmax = max(max(sh.u32[8], sh.u32[9]), max(sh.u32[10], sh.u32[11]));
        const uint32_t bmin = min(min(sh.u32[12], sh.u32[13]), min(sh.u32[14], sh.u32[15]));
        tau = block_kth(bmin, bmax, m,
                        [&](auto&& f) {
#pragma unroll
                            for (int g = 0; g < NG; ++g) f(order_key(gm[g]));
                        },
                        sh);
    }
    // tau <= kKeyNaN: fewer than m real logits in some wave; no pruning.
    const bool allpass = tau <= kKeyNaN;
    if (allpass && cend - c0 > kStage) {
        return chunk_slow_raw<T, EPT, 0>(rc, c0, m, pbits, sh, slot, stride, n_top, n_out, ok);
    }
    const float floor_v = key_value(max(tau, kKeyNegInf));  // raw >= floor_v <=> key >= tau

    // With a penalty below 1, the penalty bits of this thread's slots (bit s
    //    = slot s) select candidates: read them once (the W elements of a
    //    16-byte group lie in one bitmap word).
    uint64_t pm = 0ull;
    if (pen_all) {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int off = (v * kBlock + tid) * W;  // element offset in the chunk
            pm |= static_cast<uint64_t>((pbits[off >> 5] >> (off & 31)) & ((1u << W) - 1u)) << (v * W);
        }
    }

    // 4. Stage the candidates from ballots into this wave's segment, as
    //    (value bits << 32 | element index): the fewest instructions per
    //    candidate on this serial path. Their raw entries (order key, penalty
    //    flag) are built where they are read, one candidate per lane. A group
    //    of 4 slots is examined only if its maximum reaches the bound; with a
    //    penalty below 1 every penalised token is a candidate. A position
    //    past the segment is clamped to its last word: the count then shows
    //    the overflow and the exact routine takes over.
    const int ebase = c0 + tid * W;
    uint32_t woff = 0;  // wave-uniform
    uint64_t* seg = sh.stage + wave * kSeg;
    auto put = [&](bool c, int s) {
        const uint64_t mk = __ballot(c);
        if (mk) {
            if (c) {
                const uint32_t o = min(woff + lanes_below(mk), static_cast<uint32_t>(kSeg - 1));
                const uint32_t e = static_cast<uint32_t>(ebase + (s / W) * kBlock * W + s % W);
                seg[o] = (static_cast<uint64_t>(f2u(value(s))) << 32) | e;
            }
            woff += static_cast<uint32_t>(__popcll(mk));
        }
    };
    // The raw entry of a staged candidate.
    auto entry_of = [&](uint64_t y) -> uint64_t {
        const uint32_t e = static_cast<uint32_t>(y);
        bool pen = false;
        if (rc.pen) {
            const uint32_t off = e - static_cast<uint32_t>(c0);
            pen = ((pbits[off >> 5] >> (off & 31)) & 1u) != 0u;
        }
        return raw_entry(order_key(u2f(static_cast<uint32_t>(y >> 32))), e, pen);
    };
    if (allpass) {
#pragma unroll
        for (int s = 0; s < EPT; ++s) put(((vmask >> s) & 1ull) != 0ull, s);
    } else if (!pen_all) {
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            if (__ballot(gm[g] >= floor_v) == 0ull) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) put(value(4 * g + j) >= floor_v, 4 * g + j);
        }
    } else {
#pragma unroll
        for (int s = 0; s < EPT; ++s) put(value(s) >= floor_v || ((pm >> s) & 1ull) != 0ull, s);
    }
    fence_words();
    if (lane == 0) sh.u32[kSegCount + wave] = woff;
    __syncthreads();
    uint32_t cnt[kBlock / 64];
    uint32_t n_c = 0;
    bool seg_over = false;
#pragma unroll
    for (int w = 0; w < kBlock / 64; ++w) {
        cnt[w] = sh.u32[kSegCount + w];
        n_c += cnt[w];
        seg_over |= cnt[w] >= static_cast<uint32_t>(kSeg);
    }
    if (seg_over) {
        // Massive ties or a loose bound: the exact routine.
        return chunk_slow_raw<T, EPT, 0>(rc, c0, m, pbits, sh, slot, stride, n_top, n_out, ok);
    }
    if (n_c <= 64u && !pen_all && !ll.fs) {
        // 5. The usual case: wave 0 ranks the candidates by counting (exact
        //    64-bit keys read in pairs from LDS broadcasts, four pairs per
        //    step) and writes the sorted top m straight to the slot; the
        //    other waves go on to the ticket.
        n_top = min(n_c, m);
        n_out = n_top;
        direct = true;
        uint64_t g = 0ull;
        uint32_t rank = 0xffffffffu;
        if (wave == 0) {
            const uint32_t b1 = cnt[0], b2 = b1 + cnt[1], b3 = b2 + cnt[2];
            const uint32_t i = static_cast<uint32_t>(lane);
            const int w = (i >= b1 ? 1 : 0) + (i >= b2 ? 1 : 0) + (i >= b3 ? 1 : 0);
            const uint32_t base = w == 0 ? 0u : (w == 1 ? b1 : (w == 2 ? b2 : b3));
            const uint64_t x = i < n_c ? entry_of(sh.stage[w * kSeg + (i - base)]) : 0ull;
            sh.top[lane] = x;  // scratch (unused by the chunk phase); zeros past n_c
            wave_lds_sync();
            const ulonglong2* p2 = reinterpret_cast<const ulonglong2*>(sh.top);
            uint32_t r = 0;
            for (uint32_t j = 0; j < (n_c + 7u) / 8u; ++j) {
                const ulonglong2 q0 = p2[4 * j + 0], q1 = p2[4 * j + 1], q2 = p2[4 * j + 2], q3 = p2[4 * j + 3];
                r = add_greater4(r, q0.x, q0.y, q1.x, q1.y, x);
                r = add_greater4(r, q2.x, q2.y, q3.x, q3.y, x);
            }
            if (i < n_c && r < m) store_shared(&slot[2u + r], x);
            const uint64_t hm = __ballot(i < n_c && r == m - 1u);
            if (hm) g = wave::readlane64(x, __ffsll(static_cast<unsigned long long>(hm)) - 1);
            rank = r;
        } else if (ll.on && wave == 1) {
            // The candidates' final keys and capped raw keys, while wave 0
            // ranks them (same candidate order as wave 0's lanes).
            const uint32_t b1 = cnt[0], b2 = b1 + cnt[1], b3 = b2 + cnt[2];
            const uint32_t i = static_cast<uint32_t>(lane);
            if (i < n_c) {
                const int w = (i >= b1 ? 1 : 0) + (i >= b2 ? 1 : 0) + (i >= b3 ? 1 : 0);
                const uint32_t base = w == 0 ? 0u : (w == 1 ? b1 : (w == 2 ? b2 : b3));
                const uint64_t e = entry_of(sh.stage[w * kSeg + (i - base)]);
                const float f = softcap(key_value(static_cast<uint32_t>(e >> 32)), rc.cap);
                sh.hist[i] = order_key((rc.pen && raw_entry_pen(e)) ? penalize(f, rc.r) : f);
                sh.hist[64u + i] = order_key(f);
            }
        }
        if (ll.on) {
            __syncthreads();
            if (wave == 0 && static_cast<uint32_t>(lane) < n_c) {
                if (rank < m) store_shared(&slot[ll.fin + rank], static_cast<uint64_t>(sh.hist[lane]));
                if (rank == ll.j1 - 1u) store_shared(&slot[ll.bound], static_cast<uint64_t>(sh.hist[64 + lane]));
            }
        }
        return g;  // meaningful in wave 0, which publishes it
    }
    // 5. The top m, sorted. Up to kBlock candidates: each wave moves its
    //    segment to its place in stage[0, n_c) (inside segment 0's area past
    //    wave 0's entries, so no wave overwrites another's unread entries),
    //    then rank by counting. More: gather and sort.
    if (ll.fs && n_c <= static_cast<uint32_t>(kBlock)) {
        // Final-order list straight from the candidates: their final
        // composite keys, each ranked among all of them, the top m written to
        // the slot. The bounds are the m-th and j1-th final keys, raised to
        // the capped value of tau, which bounds every element below it (a
        // penalised candidate's final can fall below those). The softcap is
        // monotone, so without penalties these are the capped values of the
        // m-th and j1-th raw entries.
        uint32_t base = 0;
#pragma unroll
        for (int w = 0; w < kBlock / 64; ++w) base += w < wave ? cnt[w] : 0u;
        for (uint32_t i = lane; i < cnt[wave]; i += 64) {
            const uint64_t e = entry_of(seg[i]);
            const float f = softcap(key_value(static_cast<uint32_t>(e >> 32)), rc.cap);
            sh.stage[base + i] =
                composite(order_key((rc.pen && raw_entry_pen(e)) ? penalize(f, rc.r) : f), raw_entry_index(e));
        }
        if (static_cast<uint32_t>(tid) >= n_c && static_cast<uint32_t>(tid) < ((n_c + 7u) & ~7u))
            sh.stage[tid] = 0ull;
        __syncthreads();
        const bool all_listed = allpass && n_c <= m;
        const uint32_t listed = all_listed ? n_c : m;
        const uint32_t ktau = allpass ? 0u : order_key(softcap(floor_v, rc.cap));
        if (static_cast<uint32_t>(tid) < n_c) {
            const uint64_t fc = sh.stage[tid];
            const ulonglong2* p2 = reinterpret_cast<const ulonglong2*>(sh.stage);
            uint32_t r0 = 0, r1 = 0;
            for (uint32_t j = 0; j < (n_c + 7u) / 8u; ++j) {
                const ulonglong2 q0 = p2[4 * j + 0], q1 = p2[4 * j + 1], q2 = p2[4 * j + 2], q3 = p2[4 * j + 3];
                r0 = add_greater4(r0, q0.x, q0.y, q1.x, q1.y, fc);
                r1 = add_greater4(r1, q2.x, q2.y, q3.x, q3.y, fc);
            }
            const uint32_t r = r0 + r1;
            if (r < m) store_shared(&slot[2u + r], fc);
            if (r == m - 1u) sh.u32[24] = max(composite_key(fc), ktau);
            if (r == ll.j1 - 1u) sh.u32[25] = max(composite_key(fc), ktau);
        }
        if (tid == 0 && n_c < ll.j1) sh.u32[25] = 0u;  // (all listed; the header then writes 0)
        n_top = listed;
        n_out = listed;
        direct = true;
        return all_listed ? 0ull : 1ull;  // 1: a nonzero guarantee, the bounds are in sh.u32[24], [25]
    }
    if (n_c <= static_cast<uint32_t>(kBlock)) {
        uint32_t base = 0;
#pragma unroll
        for (int w = 0; w < kBlock / 64; ++w) base += w < wave ? cnt[w] : 0u;
        for (uint32_t i = lane; i < cnt[wave]; i += 64) sh.stage[base + i] = entry_of(seg[i]);
        if (static_cast<uint32_t>(tid) >= n_c && static_cast<uint32_t>(tid) < ((n_c + 7u) & ~7u))
            sh.stage[tid] = 0ull;
        __syncthreads();
        n_top = rank_top_exact(sh.stage, n_c, m, sh.list);
    } else {
        for (uint32_t i = lane; i < cnt[wave]; i += 64) seg[i] = entry_of(seg[i]);
        __syncthreads();
        seg_gather(sh.stage, cnt, n_c);
        n_top = select_top(sh.stage, n_c, m, sh.list);
    }
    n_out = n_top;
    // Elements below tau are below the m-th entry; all-pass chunks with at
    // most m elements listed everything.
    const uint64_t g = n_top == m ? sh.list[m - 1] : 0ull;
    if (pen_all && n_c > m) n_out += append_penalised(sh, n_c, m, g, slot, stride, ok);
    return ok ? g : kGuaranteeFailed;
}

__device__ __forceinline__ void write_row(const DevArgs& a, int row, int32_t token, float prob,
                                          int32_t flags) {
    emit_row(a, row, token, prob, flags);
    a.tickets[row] = 0u;  // ready for the next launch
}

// The 16 floats p[0, 16) (16-byte aligned, in LDS) in every lane: four
// broadcast 16-byte reads issued together. The sequential chains add them as
// VGPR operands, so no step waits on a v_readlane.
struct F16 {
    float v[16];
};
__device__ __forceinline__ F16 lds16(const float* p) {
    const float4* q = reinterpret_cast<const float4*>(p);
    const float4 a = q[0], b = q[1], c = q[2], d = q[3];
    return F16{{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c.x, c.y, c.z, c.w, d.x, d.y, d.z, d.w}};
}

// generation.cpp:103-126 on probabilities sorted by value desc / index asc,
// evaluated by one whole wave, for any values (NaN included). seg_prob(g)
// returns this lane's probability of entry g * 64 + lane (0 past keff). Every
// lane computes the same sequential fp32 (and, for the boundary distances,
// double) chain; lane j keeps step j of each 64-entry segment (a select), so
// each stop test is one ballot.
template <typename P>
__device__ __forceinline__ void scan_and_walk(P&& seg_prob, uint32_t keff, const ge_sample_params& p,
                                              float u, uint32_t& pos_out, bool& near_out) {
    const int lane = __lane_id();
    const float minimum = readlane_f(seg_prob(0u), 0) * p.min_p;
    float cum = 0.0f;
    float mass = 0.0f;
    uint32_t keep = keff;
    bool stopped = false;
    const uint32_t nseg = (keff + 63) / 64;
    for (uint32_t g = 0; g < nseg && !stopped; ++g) {
        const float pl = seg_prob(g);
        const float before = cum;
        float cl = 0.0f;
        for (int q = 0; q < 64; q += 16) {
            static_for<0, 16>([&](auto J) {
                cum = cum + readlane_f(pl, q + J);
                cl = lane == q + J ? cum : cl;
            });
        }
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
    if (!stopped) mass = cum;  // entries past keff add exact zeros
    const float choice0 = u * mass + 0.0f;  // uniform_real_distribution(0, mass)
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
        for (int q = 0; q < 64; q += 16) {
            static_for<0, 16>([&](auto J) {
                const float pj = readlane_f(pl, q + J);
                choice = choice - pj;
                dc = dc + static_cast<double>(pj);
                chl = lane == q + J ? choice : chl;
                dl = lane == q + J ? dc : dl;
            });
        }
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

// The same chains when no probability is NaN. Then the probabilities are
// non-increasing (expf is monotone and the values are sorted), so the min-p
// cut is one parallel search and the cumulative / choice chains are
// monotone. Every lane runs the reference's sequential fp32 adds, 64 steps per
// segment, with the step's probability broadcast from the lane holding it
// (v_readlane, off the add chain); lane i keeps the sum after step i (a
// v_cndmask, also off the chain), so one ballot finds the stop in a segment.
// seg_prob(g) returns this lane's probability of entry g * 64 + lane (any
// finite value past keff; those entries are masked here).
template <typename P>
__device__ __forceinline__ void scan_and_walk_fast(P&& seg_prob, const float* probs, uint32_t keff,
                                                   const ge_sample_params& p, float u, uint32_t& pos_out,
                                                   bool& near_out) {
    const int lane = __lane_id();
    const float p0 = readlane_f(seg_prob(0u), 0);
    const float minimum = p0 * p.min_p;
    // min-p: first j >= 1 with p_j < minimum (checked before adding p_j);
    // none when minimum <= 0 (probabilities are >= 0).
    uint32_t limit = keff;
    if (minimum > 0.0f) {
        for (uint32_t g = 0; g * 64 < keff; ++g) {
            const uint32_t j = g * 64 + static_cast<uint32_t>(lane);
            const uint64_t h = __ballot(j >= 1 && j < keff && seg_prob(g) < minimum);
            if (h) {
                limit = g * 64 + static_cast<uint32_t>(__ffsll(static_cast<unsigned long long>(h)) - 1);
                break;
            }
        }
    }
    // top-p: first j >= 1, j < limit, with cum_j >= top_p. The chain runs in
    // blocks of 16 plain adds, fully unrolled; cum is non-decreasing, so the
    // stop lies in the first block that ends at or above top_p, which is then
    // replayed from its starting value (same adds, same bits) with lane j
    // keeping the sum after step j, and one ballot finds it.
    float cum = 0.0f;
    float mass = 0.0f;
    uint32_t keep = limit;
    bool stopped = false;
    for (uint32_t g = 0; g * 64 < limit && !stopped; ++g) {
        const uint32_t idx = g * 64 + static_cast<uint32_t>(lane);
        const float pl = idx < limit ? seg_prob(g) : 0.0f;
        // A whole segment below the limit: its 64 probabilities are read
        // together (sixteen broadcast 16-byte reads in flight), so the chain
        // waits for LDS once per 64 steps.
        const bool whole = g * 64 + 64 <= limit;
        F16 qs[4];
        if (whole) static_for<0, 4>([&](auto B) { qs[decltype(B)::value] = lds16(probs + g * 64 + decltype(B)::value * 16); });
        static_for<0, 4>([&](auto B) {
            constexpr int b = decltype(B)::value * 16;
            if (stopped) return;
            const float before = cum;
            if (whole) {
                static_for<0, 16>([&](auto J) { cum = cum + qs[decltype(B)::value].v[decltype(J)::value]; });
            } else if (g * 64 + b + 16 <= limit) {
                const F16 q = lds16(probs + g * 64 + b);  // whole block below the limit
                static_for<0, 16>([&](auto J) { cum = cum + q.v[decltype(J)::value]; });
            } else {
                static_for<0, 16>([&](auto J) { cum = cum + readlane_f(pl, b + decltype(J)::value); });
            }
            if (cum >= p.top_p) {
                float c = before, cl = 0.0f;
                static_for<0, 16>([&](auto J) {
                    constexpr int j = b + decltype(J)::value;
                    c = c + readlane_f(pl, j);
                    cl = put_lane<j>(cl, c);
                });
                const uint64_t th = __ballot(lane >= b && lane < b + 16 && idx >= 1 && idx < limit && cl >= p.top_p);
                if (th) {
                    const int j = __ffsll(static_cast<unsigned long long>(th)) - 1;
                    keep = g * 64 + static_cast<uint32_t>(j) + 1u;
                    mass = readlane_f(cl, j);
                    stopped = true;
                }
            }
        });
    }
    if (!stopped) mass = cum;  // min-p cut or all keff kept
    // Draw: uniform_real_distribution(0, mass), then the subtract walk
    // (choice is non-increasing: the same block search).
    const float choice0 = u * mass + 0.0f;
    float choice = choice0;
    uint32_t pos = keep - 1;  // fallthrough return, generation.cpp:126
    bool found = false;
    for (uint32_t g = 0; g * 64 < keep && !found; ++g) {
        const uint32_t idx = g * 64 + static_cast<uint32_t>(lane);
        const float pl = idx < keep ? seg_prob(g) : 0.0f;
        const bool whole = g * 64 + 64 <= keep;
        F16 qs[4];
        if (whole) static_for<0, 4>([&](auto B) { qs[decltype(B)::value] = lds16(probs + g * 64 + decltype(B)::value * 16); });
        static_for<0, 4>([&](auto B) {
            constexpr int b = decltype(B)::value * 16;
            if (found) return;
            const float before = choice;
            if (whole) {
                static_for<0, 16>([&](auto J) { choice = choice - qs[decltype(B)::value].v[decltype(J)::value]; });
            } else if (g * 64 + b + 16 <= keep) {
                const F16 q = lds16(probs + g * 64 + b);
                static_for<0, 16>([&](auto J) { choice = choice - q.v[decltype(J)::value]; });
            } else {
                static_for<0, 16>([&](auto J) { choice = choice - readlane_f(pl, b + decltype(J)::value); });
            }
            if (choice <= 0.0f) {
                float c = before, cl = 0.0f;
                static_for<0, 16>([&](auto J) {
                    constexpr int j = b + decltype(J)::value;
                    c = c - readlane_f(pl, j);
                    cl = put_lane<j>(cl, c);
                });
                const uint64_t hit = __ballot(lane >= b && lane < b + 16 && idx < keep && cl <= 0.0f);
                if (hit) {
                    pos = g * 64 + static_cast<uint32_t>(__ffsll(static_cast<unsigned long long>(hit)) - 1);
                    found = true;
                }
            }
        });
    }
    // The reference's boundary sums: c_at = sum_{i <= pos} (double)p_i in
    // order, c_before the same up to pos - 1. A wave prefix sum gives them
    // exactly when every term is a multiple of 2^L with L >= -52 (all partial
    // sums are below 2, so 53 bits hold them in any order); else replay.
    double c_before = 0.0, c_at = 0.0;
    {
        const uint32_t gp = pos / 64;
        double base = 0.0;
        int lmin = INT_MAX;
        for (uint32_t g = 0; g <= gp; ++g) {
            const uint32_t idx = g * 64 + static_cast<uint32_t>(lane);
            const float pl = idx <= pos ? seg_prob(g) : 0.0f;
            if (pl > 0.0f) lmin = min(lmin, lsb_exponent(pl));
        }
        lmin = wave_min_i(lmin);
        if (lmin >= -52) {
            for (uint32_t g = 0; g <= gp; ++g) {
                const uint32_t idx = g * 64 + static_cast<uint32_t>(lane);
                const float pl = idx <= pos ? seg_prob(g) : 0.0f;
                const double incl = base + wave_incl_f64(static_cast<double>(pl));
                if (g == gp) {
                    const int at = static_cast<int>(pos - g * 64);
                    c_at = readlane_d(incl, at);
                    c_before = at > 0 ? readlane_d(incl, at - 1) : base;
                }
                base = readlane_d(incl, 63);
            }
        } else {
            double dc = 0.0;
            for (uint32_t g = 0; g <= gp; ++g) {
                const float pl = seg_prob(g);
                const int last = g == gp ? static_cast<int>(pos - g * 64) : 63;
                for (int i = 0; i <= last; ++i) {
                    c_before = dc;
                    dc = dc + static_cast<double>(readlane_f(pl, i));
                }
            }
            c_at = dc;
        }
    }
    bool near = false;
    if (pos > 0 && fabs(static_cast<double>(choice0) - c_before) < 1e-6) near = true;
    if (pos + 1 < keep && fabs(static_cast<double>(choice0) - c_at) < 1e-6) near = true;
    pos_out = pos;
    near_out = near;
}


// generation.cpp:103-126 for at most 64 probabilities in one wave's
// registers (lane j holds p_j, j < keff; none NaN, so they are
// non-increasing). The sequential fp32 sums are fully unrolled in blocks of
// 16 steps: every lane runs the same chain with p_j broadcast from LDS, lane
// j keeps the sum after step j, and one ballot per block finds the stop, with
// no replay and no per-step branch. The draw's walk runs over the same LDS
// copy (the min-p-masked values; it never looks past keep - 1, so the
// entries past keep need no masking) and reuses block 0's broadcast. The
// double boundary sums come from a wave prefix sum of the same values when it
// is exact (every term a multiple of 2^-52; the partial sums are below 2),
// else from a sequential replay; both are independent of the chains.
__device__ __forceinline__ void scan_walk_wave(float pr, uint32_t keff, const ge_sample_params& p, float u,
                                               float* lds, uint32_t& pos_out, bool& near_out) {
    const int lane = __lane_id();
    const float p0 = readlane_f(pr, 0);
    const float minimum = p0 * p.min_p;
    // min-p: the first j >= 1 with p_j < minimum (checked before adding p_j).
    uint32_t limit = keff;
    if (minimum > 0.0f) {
        const uint64_t h = __ballot(lane >= 1 && lane < static_cast<int>(keff) && pr < minimum);
        if (h) limit = static_cast<uint32_t>(__ffsll(static_cast<unsigned long long>(h)) - 1);
    }
    // top-p: the first j in [1, limit) with cum_j >= top_p. Entries past the
    // limit add exact zeros.
    const float pl = lane < static_cast<int>(limit) ? pr : 0.0f;
    lds[lane] = pl;
    // Boundary sums (positions up to pos < keep <= limit only): exact wave
    // prefix when every term of the limit's prefix is a multiple of 2^-52;
    // computed in the shadow of block 0's LDS read.
    bool incl_exact = false;
    double incl = 0.0;
    float cum = 0.0f, mass = 0.0f, cl = 0.0f;
    uint32_t keep = limit;
    bool stopped = false;
    F16 q0;
    static_for<0, 4>([&](auto B) {
        constexpr int b = decltype(B)::value * 16;
        if (stopped || static_cast<uint32_t>(b) >= limit) return;
        const F16 q = lds16(lds + b);
        if constexpr (b == 0) {
            q0 = q;
            incl_exact = wave_min_i(pl > 0.0f ? lsb_exponent(pl) : INT_MAX) >= -52;
            incl = wave_incl_f64(static_cast<double>(pl));
        }
        static_for<0, 16>([&](auto J) {
            constexpr int j = b + decltype(J)::value;
            cum = cum + q.v[decltype(J)::value];
            cl = put_lane<j>(cl, cum);
        });
        const uint64_t th = __ballot(lane >= b && lane < b + 16 && lane >= 1 && lane < static_cast<int>(limit) &&
                                     cl >= p.top_p);
        if (th) {
            const int j = __ffsll(static_cast<unsigned long long>(th)) - 1;
            keep = static_cast<uint32_t>(j) + 1u;
            mass = readlane_f(cl, j);
            stopped = true;
        }
    });
    if (!stopped) mass = cum;
    // Draw: uniform_real_distribution(0, mass), then the subtract walk; the
    // fall-through returns entry keep - 1 (generation.cpp:126).
    const float choice0 = u * mass + 0.0f;
    float choice = choice0, chl = 0.0f;
    uint32_t pos = keep - 1u;
    bool found = false;
    static_for<0, 4>([&](auto B) {
        constexpr int b = decltype(B)::value * 16;
        if (found || static_cast<uint32_t>(b) >= keep) return;
        F16 q;
        if constexpr (b == 0) q = q0;
        else q = lds16(lds + b);
        static_for<0, 16>([&](auto J) {
            constexpr int j = b + decltype(J)::value;
            choice = choice - q.v[decltype(J)::value];
            chl = put_lane<j>(chl, choice);
        });
        const uint64_t hit = __ballot(lane >= b && lane < b + 16 && lane < static_cast<int>(keep) && chl <= 0.0f);
        if (hit) {
            pos = static_cast<uint32_t>(__ffsll(static_cast<unsigned long long>(hit)) - 1);
            found = true;
        }
    });
    double c_before = 0.0, c_at = 0.0;
    if (incl_exact) {
        c_at = readlane_d(incl, static_cast<int>(pos));
        c_before = pos > 0 ? readlane_d(incl, static_cast<int>(pos) - 1) : 0.0;
    } else {
        double dc = 0.0;
        for (uint32_t i = 0; i <= pos; ++i) {
            c_before = dc;
            dc = dc + static_cast<double>(readlane_f(pl, static_cast<int>(i)));
        }
        c_at = dc;
    }
    bool near = false;
    if (pos > 0 && fabs(static_cast<double>(choice0) - c_before) < 1e-6) near = true;
    if (pos + 1 < keep && fabs(static_cast<double>(choice0) - c_at) < 1e-6) near = true;
    pos_out = pos;
    near_out = near;
}

// Rank by counting over per-wave segments, each padded with zero keys to a
// multiple of 8 (four 16-byte broadcast reads per step); also stores term(x),
// computed alongside the count, at ex[rank] for ranks below m.
template <typename Term>
__device__ __forceinline__ void seg_rank_expf(const uint64_t* stage, const uint32_t (&cnt)[kBlock / 64], uint32_t n,
                                              uint32_t m, uint64_t* dst, Term&& term, float* ex) {
    const int tid = threadIdx.x;
    if (static_cast<uint32_t>(tid) < n) {
        int w = 0;
        uint32_t i = static_cast<uint32_t>(tid);
        while (i >= cnt[w]) {
            i -= cnt[w];
            ++w;
        }
        const uint64_t x = stage[w * kSeg + i];
        const float t = term(x);  // independent of the rank: overlaps it
        uint32_t rk = 0;
#pragma unroll
        for (int v = 0; v < kBlock / 64; ++v) {
            const ulonglong2* p2 = reinterpret_cast<const ulonglong2*>(stage + v * kSeg);
            for (uint32_t j = 0; j < (cnt[v] + 7u) / 8u; ++j) {
                const ulonglong2 q0 = p2[4 * j + 0], q1 = p2[4 * j + 1], q2 = p2[4 * j + 2], q3 = p2[4 * j + 3];
                rk = add_greater4(rk, q0.x, q0.y, q1.x, q1.y, x);
                rk = add_greater4(rk, q2.x, q2.y, q3.x, q3.y, x);
            }
        }
        if (rk < m) {
            dst[rk] = x;
            ex[rk] = t;
        }
    }
    __syncthreads();
}

// sh.top[0, nt) := the largest k distinct keys of sh.top[0, nt) and
// sh.list[0, nl), sorted descending. Returns the new nt. Block-uniform.
__device__ __forceinline__ uint32_t absorb_list(SelShared& sh, uint32_t nt, uint32_t nl, uint32_t k) {
    const int tid = threadIdx.x;
    const uint32_t n = nt + nl;
    for (uint32_t i = tid; i < nt; i += kBlock) sh.stage[i] = sh.top[i];
    for (uint32_t i = tid; i < nl; i += kBlock) sh.stage[nt + i] = sh.list[i];
    uint32_t n2 = 1;
    while (n2 < n) n2 <<= 1;
    for (uint32_t i = n + tid; i < n2; i += kBlock) sh.stage[i] = 0ull;
    __syncthreads();
    bitonic_desc_block(sh.stage, n2);
    // Drop duplicates (a key present in both lists) and zeros; keep k.
    uint32_t kept_total = 0;
    for (uint32_t base = 0; base < n; base += kBlock) {
        const uint32_t i = base + tid;
        const uint64_t x = i < n ? sh.stage[i] : 0ull;
        const bool keep = i < n && x != 0ull && (i == 0 || sh.stage[i - 1] != x);
        uint32_t total;
        const uint32_t pos = kept_total + block_excl_scan(keep ? 1u : 0u, total, sh);
        if (keep && pos < k) sh.top[pos] = x;
        kept_total += total;
    }
    __syncthreads();
    return min(kept_total, k);
}

// Loads the row's slot words, kPer per thread: w[i], its position wp[i] in
// its chunk's slot (0 = the guarantee, 1 = the count, 2.. = entries; past the
// end: 0xffffffff) and its chunk wc[i]; stores each chunk's guarantee in
// sh.gam[c] and its count in sh.cnt[c], and stages the expf table in
// sh.exp_tab. One round trip. After a barrier,
// slot_entry(...) tells which words are entries of this launch (a chunk's
// words past its count hold older data).
template <int kPer>
__device__ __forceinline__ void load_slots(const DevArgs& a, SelShared& sh, int row, uint32_t stride,
                                           uint64_t (&w)[kPer], uint32_t (&wp)[kPer], uint32_t (&wc)[kPer]) {
    const int tid = threadIdx.x;
    const uint32_t words = static_cast<uint32_t>(a.cpr) * stride;  // <= kSlotWords
    const uint64_t* slot_row = a.slots + static_cast<int64_t>(row) * kSlotWords;
    // All loads first (independent round trips in flight together), then the
    // LDS writes that need their results. The loads are unconditional (words
    // past the slots read the last word and are then dropped): a load under
    // a lane mask is followed by a wait for every load in flight.
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const uint32_t g = static_cast<uint32_t>(i * kBlock + tid);
        w[i] = load_shared(&slot_row[min(g, words - 1u)]);
    }
    // The expf table (2^(i/32)) from constant memory, in flight with the
    // lists (a wait for it alone would delay their issue by a round trip).
    const uint64_t et = exp2_table(static_cast<uint32_t>(tid) & 31u);
#pragma unroll
    for (int i = 0; i < kPer; ++i)
        if (static_cast<uint32_t>(i * kBlock + tid) >= words) w[i] = 0ull;
    uint32_t c = static_cast<uint32_t>(tid) / stride, q = static_cast<uint32_t>(tid) % stride;
    const uint32_t dc = kBlock / stride, dq = kBlock % stride;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const uint32_t g = static_cast<uint32_t>(i * kBlock + tid);
        wp[i] = g < words ? q : 0xffffffffu;
        wc[i] = c;
        c += dc;
        q += dq;
        if (q >= stride) {
            q -= stride;
            ++c;
        }
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        if (wp[i] == 0u) sh.gam[wc[i]] = w[i];
        if (wp[i] == 1u) sh.cnt[wc[i]] = static_cast<uint32_t>(w[i]);
    }
    if (tid < 32) sh.exp_tab[tid] = et;
}

// LDS *p = max(*p, v), one ds_max_u64 per lane. Written out because the
// compiler's atomic optimizer turns an atomicMax on one LDS address from
// divergent lanes into a serial loop over the active lanes (readlane per
// lane). Not ordered by the compiler: callers wait (lds_wait) before the
// barrier that publishes the result.
__device__ __forceinline__ void lds_max_u64(uint64_t* p, uint64_t v) {
    const uint32_t addr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint64_t*)p));
    asm volatile("ds_max_u64 %0, %1" ::"v"(addr), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_wait() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// After the barrier that follows load_slots (sh.u64[0..1] cleared before
// it): which loaded words are entries of this launch (ent[i]; a chunk's words
// past its count hold older data), and the row's largest guarantees, at
// level m each chunk's guarantee word and at level j1 each chunk's j1-th
// entry (every element outside a chunk's first j1 entries is below it). A
// chunk that listed fewer than j1 entries listed everything and adds
// nothing; a chunk that failed makes both levels fail. The lanes holding
// those words fold them into LDS with atomicMax: no cross-lane reduction.
// kLevel1 = false: level m only (g1 = 0). Block-uniform (one barrier).
template <bool kLevel1, int kPer>
__device__ __forceinline__ void row_guarantees(SelShared& sh, uint32_t j1, const uint64_t (&w)[kPer],
                                               const uint32_t (&wp)[kPer], const uint32_t (&wc)[kPer],
                                               bool (&ent)[kPer], uint64_t& gm, uint64_t& g1) {
    uint32_t cn[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) cn[i] = wp[i] != 0xffffffffu ? sh.cnt[wc[i]] : 0u;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        ent[i] = wp[i] >= 2u && wp[i] != 0xffffffffu && wp[i] - 2u < cn[i];
        if (wp[i] == 0u && w[i] != 0ull) lds_max_u64(&sh.u64[0], w[i]);
        if (kLevel1 && wp[i] == 1u + j1) {
            const uint64_t g = sh.gam[wc[i]];
            const uint64_t v = g == kGuaranteeFailed ? kGuaranteeFailed : (cn[i] >= j1 ? w[i] : 0ull);
            if (v != 0ull) lds_max_u64(&sh.u64[1], v);
        }
    }
    lds_wait();
    __syncthreads();
    gm = sh.u64[0];
    g1 = sh.u64[1];
}

__device__ __forceinline__ bool slot_entry(const SelShared& sh, uint32_t wp, uint32_t wc) {
    return wp >= 2u && wp != 0xffffffffu && wp - 2u < sh.cnt[wc];
}

// Final composite key of a raw list entry: softcap, then the penalty if the
// entry is penalised.
__device__ __forceinline__ uint64_t final_of(uint64_t e, const RowCtx& rc) {
    float f = softcap(key_value(static_cast<uint32_t>(e >> 32)), rc.cap);
    if (rc.pen && raw_entry_pen(e)) f = penalize(f, rc.r);
    return composite(order_key(f), raw_entry_index(e));
}

// Merge, first part (last workgroup of the row), one round trip for every
// chunk's guarantee and list. With G the largest guarantee, every element
// whose raw entry is > G is listed, and every other element ends at most at
// C = softcap(value of G). The merge caps and penalises the listed entries
// above G (with a penalty below 1, also every listed penalised entry), takes
// their top k by final value into sh.top[0, nt) and returns true when that is
// certified to be the row's top k: the k-th final value is above C (so no
// element outside can reach it or tie with it), or every chunk listed
// everything. Otherwise returns false (a chunk held more of the top k than it
// listed, or a tie at the bound): the caller falls back to merge_all_lists.
__device__ __forceinline__ bool merge_collect(const DevArgs& a, SelShared& sh, const RowCtx& rc, uint32_t k,
                                              uint32_t stride, uint32_t& nt) {
    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int wave = tid >> 6;
    constexpr int kPer = kSlotWords / kBlock;
    uint64_t w[kPer];
    uint32_t wp[kPer], wc[kPer];
    if (tid == 0) sh.u64[0] = sh.u64[1] = 0ull;
    load_slots(a, sh, rc.row, stride, w, wp, wc);
    __syncthreads();
    uint64_t gam_max, gam1;
    bool ent[kPer];
    row_guarantees<false>(sh, 1u, w, wp, wc, ent, gam_max, gam1);
    const bool bounded = gam_max != 0ull && gam_max != kGuaranteeFailed;
    const bool pen_all = rc.pen && !(rc.r >= 1.0f);

    // The entries above the largest guarantee, staged in per-wave segments.
    uint64_t* seg = sh.stage + wave * kSeg;
    {
        uint32_t woff = 0;  // <= kPer * 64 = kSeg
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const bool c = ent[i] && (w[i] > gam_max || (pen_all && raw_entry_pen(w[i])));
            const uint64_t mk = __ballot(c);
            if (c) seg[woff + lanes_below(mk)] = w[i];
            woff += static_cast<uint32_t>(__popcll(mk));
        }
        if (lane == 0) {
            sh.u32[kSegCount + wave] = woff;
            if ((woff & 1u) && woff < static_cast<uint32_t>(kSeg)) seg[woff] = 0ull;
        }
    }
    __syncthreads();
    uint32_t cnt[kBlock / 64];
    uint32_t nsel = 0;
#pragma unroll
    for (int v = 0; v < kBlock / 64; ++v) {
        cnt[v] = sh.u32[kSegCount + v];
        nsel += cnt[v];
    }
    // Final values in place, each wave over its own segment; wave 0 caps the
    // largest guarantee's raw value as one more item of the same pass.
    {
        const uint32_t n = cnt[wave] + ((wave == 0 && bounded) ? 1u : 0u);
        for (uint32_t i = lane; i < n; i += 64) {
            const bool real = i < cnt[wave];
            const uint64_t e = real ? seg[i] : gam_max;
            float f = softcap(key_value(static_cast<uint32_t>(e >> 32)), rc.cap);
            if (real) {
                if (rc.pen && raw_entry_pen(e)) f = penalize(f, rc.r);
                seg[i] = composite(order_key(f), raw_entry_index(e));
            } else {
                sh.u32[16] = order_key(f);
            }
        }
    }
    __syncthreads();
    // Top k by final value, sorted. Few entries: rank by counting. More: a
    // radix lower bound on the k-th value key (one digit when that leaves
    // few) cuts them to about k first.
    if (nsel <= kRankDirect) {
        seg_rank_top(sh.stage, cnt, nsel, k, sh.top);
        nt = min(nsel, k);
    } else {
        constexpr int kPerW = kSeg / 64;
        uint64_t e[kPerW];
#pragma unroll
        for (int q = 0; q < kPerW; ++q) {
            const uint32_t i = static_cast<uint32_t>(q * 64 + lane);
            e[q] = i < cnt[wave] ? seg[i] : 0ull;
        }
        uint32_t kk = 0u;  // keep entries whose value key is >= kk
        if (nsel > k) {
            uint32_t kmin = 0xffffffffu, kmax = 0u;
#pragma unroll
            for (int q = 0; q < kPerW; ++q)
                if (e[q] != 0ull) {
                    kmin = min(kmin, composite_key(e[q]));
                    kmax = max(kmax, composite_key(e[q]));
                }
            kmin = wave_min(kmin);
            kmax = wave_max(kmax);
            if (lane == 0) {
                sh.u32[8 + wave] = kmax;
                sh.u32[12 + wave] = kmin;
            }
            __syncthreads();
            const uint32_t bmax = max(max(sh.u32[8], sh.u32[9]), max(sh.u32[10], sh.u32[11]));
            const uint32_t bmin = min(min(sh.u32[12], sh.u32[13]), min(sh.u32[14], sh.u32[15]));
            kk = block_kth(bmin, bmax, k,
                           [&](auto&& f) {
#pragma unroll
                               for (int q = 0; q < kPerW; ++q)
                                   if (e[q] != 0ull) f(composite_key(e[q]));
                           },
                           sh, 2u * k + 32u);
        }
        uint32_t c2 = 0;
#pragma unroll
        for (int q = 0; q < kPerW; ++q) c2 += (e[q] != 0ull && composite_key(e[q]) >= kk) ? 1u : 0u;
        // (The scan's barriers also order every wave's reads of its segment
        // before the writes below.)
        uint32_t pos = block_excl_scan(c2, nsel, sh);
#pragma unroll
        for (int q = 0; q < kPerW; ++q)
            if (e[q] != 0ull && composite_key(e[q]) >= kk) sh.stage[pos++] = e[q];
        __syncthreads();
        nt = select_top(sh.stage, nsel, k, sh.top);
    }
    if (gam_max == 0ull) return true;  // every chunk listed everything
    if (!bounded) return false;
    return nt >= k && composite_key(sh.top[k - 1]) > sh.u32[16];
}

// Words per thread of the small-row merge: rows whose slot area (cpr *
// stride words) fits kBlock * kSmallWords take merge_collect_small.
constexpr int kSmallWords = 4;

// Merge, first part, for rows with small slot areas. Same contract as
// merge_collect, fewer steps, and two levels. At level j1 (then m) with G the
// largest j1-th (m-th) list entry of the row's chunks, S = the listed entries
// above G (with a penalty below 1, also every listed penalised entry) holds
// every element whose raw entry is above G; every other element ends at most
// at C = softcap(value of G). S is compacted into sh.stage, capped and
// penalised in one balanced pass and ranked into sh.top; the top k is
// certified when its k-th final value is above C. Block-uniform.
__device__ __forceinline__ bool merge_collect_small(const DevArgs& a, SelShared& sh, const RowCtx& rc, uint32_t k,
                                                    uint32_t j1, uint32_t stride, uint32_t& nt) {
    const int tid = threadIdx.x;
    const bool pen_all = rc.pen && !(rc.r >= 1.0f);
    uint64_t w[kSmallWords];
    uint32_t wp[kSmallWords], wc[kSmallWords];
    if (tid == 0) sh.u64[0] = sh.u64[1] = 0ull;
    load_slots(a, sh, rc.row, stride, w, wp, wc);
    __syncthreads();
    // The row's largest guarantees at level j1 and at level m.
    uint64_t gam_lv[2];
    bool ent[kSmallWords];
    row_guarantees<true>(sh, j1, w, wp, wc, ent, gam_lv[1], gam_lv[0]);
    for (int lv = 0; lv < 2; ++lv) {
        const uint64_t gam = gam_lv[lv];
        if (gam == kGuaranteeFailed) return false;
        if (lv == 1 && gam == gam_lv[0]) break;  // the same bound again
        const bool bounded = gam != 0ull;
        uint32_t in = 0u, cnt = 0u;
#pragma unroll
        for (int i = 0; i < kSmallWords; ++i) {
            const bool c = ent[i] && (w[i] > gam || (pen_all && raw_entry_pen(w[i])));
            in |= static_cast<uint32_t>(c) << i;
            cnt += c ? 1u : 0u;
        }
        uint32_t n;
        uint32_t pos = block_excl_scan(cnt, n, sh);
#pragma unroll
        for (int i = 0; i < kSmallWords; ++i)
            if ((in >> i) & 1u) sh.stage[pos++] = w[i];
        __syncthreads();
        // Final values in place; item n caps G's raw value. Zeros pad the
        // entries to a multiple of 8 for the rank's paired reads.
        if (static_cast<uint32_t>(tid) >= n && static_cast<uint32_t>(tid) < ((n + 7u) & ~7u)) sh.stage[tid] = 0ull;
        const uint32_t items = n + (bounded ? 1u : 0u);
        for (uint32_t i = tid; i < items; i += kBlock) {
            const bool real = i < n;
            const uint64_t e = real ? sh.stage[i] : gam;
            float f = softcap(key_value(static_cast<uint32_t>(e >> 32)), rc.cap);
            if (real) {
                if (rc.pen && raw_entry_pen(e)) f = penalize(f, rc.r);
                sh.stage[i] = composite(order_key(f), raw_entry_index(e));
            } else {
                sh.u32[16] = order_key(f);
            }
        }
        __syncthreads();
        nt = n <= static_cast<uint32_t>(kBlock) ? rank_top_exact(sh.stage, n, k, sh.top)
                                               : select_top(sh.stage, n, k, sh.top);
        if (!bounded) return true;  // every chunk listed everything
        if (nt >= k && composite_key(sh.top[k - 1]) > sh.u32[16]) return true;
    }
    return false;
}

// Merge fallback: the top k of every listed entry by final value into
// sh.top[0, nt), and in sh.gam[c] a bound for chunk c: a composite key that
// no element the chunk left out can exceed (0: it listed everything;
// kGuaranteeFailed: it must be rescanned). Block-uniform.
__device__ __forceinline__ void merge_all_lists(const DevArgs& a, SelShared& sh, const RowCtx& rc, uint32_t k,
                                                uint32_t stride, uint32_t& nt) {
    const int tid = threadIdx.x;
    constexpr int kPer = kSlotWords / kBlock;
    uint64_t w[kPer];
    uint32_t wp[kPer], wc[kPer];
    load_slots(a, sh, rc.row, stride, w, wp, wc);
    __syncthreads();
    bool ent[kPer];
    uint32_t cnt = 0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        ent[i] = slot_entry(sh, wp[i], wc[i]);
        cnt += ent[i] ? 1u : 0u;
    }
    uint32_t n;
    uint32_t pos = block_excl_scan(cnt, n, sh);
#pragma unroll
    for (int i = 0; i < kPer; ++i)
        if (ent[i]) sh.stage[pos++] = w[i];
    __syncthreads();
    for (uint32_t i = tid; i < n; i += kBlock) sh.stage[i] = final_of(sh.stage[i], rc);
    for (int c = tid; c < a.cpr; c += kBlock) {
        const uint64_t g = sh.gam[c];
        if (g != 0ull && g != kGuaranteeFailed)
            sh.gam[c] = (static_cast<uint64_t>(order_key(softcap(key_value(static_cast<uint32_t>(g >> 32)), rc.cap)))
                         << 32) | 0xffffffffull;
    }
    __syncthreads();
    nt = select_top(sh.stage, n, k, sh.top);
}

// Next chunk at or after c whose guarantee is above the running k-th key
// (0 while fewer than k are known); -1 if none. Block-uniform.
__device__ __forceinline__ int next_rescan(const SelShared& sh, int c, int cpr, uint32_t nt, uint32_t k) {
    const uint64_t ku = nt >= k ? sh.top[k - 1] : 0ull;
    for (; c < cpr; ++c)
        if (sh.gam[c] > ku) return c;
    return -1;
}

// Merge, second part: softmax / min-p / top-p / draw over top[0, keff)
// (composite final keys, sorted descending); prob: keff floats of LDS
// scratch (at least 128) that do not overlap top.
template <typename T>
__device__ __forceinline__ void merge_finish(const DevArgs& a, SelShared& sh, const RowCtx& rc,
                                             const ge_sample_params& p, bool greedy, uint32_t keff,
                                             float u, float x0, const uint64_t* top, float* prob) {
    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int wave = tid >> 6;
    const int row = rc.row;
    if (keff == 0u) {
        if (tid == 0) write_row(a, row, -1, 0.0f, GE_FLAG_UNSUPPORTED);
        return;
    }
    if (greedy) {
        if (tid == 0) {
            // std::max_element (generation.cpp:66-70) keeps index 0 when its
            // final value is NaN (NaN < x is false): its capped value is NaN,
            // or 0 is in the history and the penalty makes it NaN (a NaN
            // penalty, -inf * 0, 0 * inf, inf / inf).
            int32_t token = static_cast<int32_t>(composite_index(top[0]));
            const float f0 = softcap(x0, rc.cap);
            bool nan0 = __builtin_isnan(f0);
            if (!nan0 && rc.pen && __builtin_isnan(penalize(f0, rc.r)))
                for (int j = 0; j < rc.H && !nan0; ++j) nan0 = rc.hist[j] == 0;
            if (nan0) token = 0;
            write_row(a, row, token, 1.0f, 0);
        }
        return;
    }

    // generation.cpp:89-101 — p_i = expf((v_i - max) * (1/T)); double denominator.
    const float maximum = key_value(composite_key(top[0]));
    const float inv_temp = 1.0f / p.temperature;
    auto expf_lds = [&](float x) { return expf_glibc_tab(x, [&](uint32_t i) { return sh.exp_tab[i]; }); };
    const bool one_wave = keff <= 64u;
    float pr_reg = 0.0f;  // one-wave path: this lane's probability
    bool any_nan;
    if (one_wave) {
        // One wave, probabilities in registers, no barriers.
        if (wave != 0) return;
        const bool live = lane < static_cast<int>(keff);
        const uint64_t c = live ? top[lane] : 0ull;
        const float e = live ? expf_lds((key_value(composite_key(c)) - maximum) * inv_temp) : 0.0f;
        const bool bad = live && (!(e >= 0.0f) || __builtin_isinf(e));
        const int lsb = (live && e > 0.0f && !bad) ? lsb_exponent(e) : INT_MAX;
        const double s = wave_sum(static_cast<double>(e));
        const int mn = wave_min_i(lsb);
        const int ex = static_cast<int>((d2u(s) >> 52) & 0x7ffu) - 1023;
        double den;
        // Certified exact (see below): any order equals the sequential sum.
        if (!__any(bad) && s > 0.0 && !__builtin_isinf(s) && mn >= ex - 51) {
            den = s;
        } else {
            den = 0.0;
            for (uint32_t i = 0; i < keff; ++i) den += static_cast<double>(readlane_f(e, static_cast<int>(i)));
        }
        const float inv_denom = static_cast<float>(1.0 / den);
        pr_reg = e * inv_denom;
        any_nan = __any(live && __builtin_isnan(pr_reg));
    } else {
        double lsum = 0.0;
        int lmin = INT_MAX;
        int bad = 0;
        for (uint32_t i = tid; i < keff; i += kBlock) {
            const float v = key_value(composite_key(top[i]));
            const float e = expf_lds((v - maximum) * inv_temp);
            prob[i] = e;
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
            int mn = INT_MAX;
            bool b = false;
            for (int wv = 0; wv < kBlock / 64; ++wv) {
                s += sh.f64[wv];
                if (sh.i32[wv] == INT_MIN) b = true;
                else mn = min(mn, sh.i32[wv]);
            }
            // Certified exact: every term is a multiple of 2^mn and every
            // partial sum is below 2^(E+2), so 53 bits hold each partial sum
            // exactly when mn >= E - 51; then any summation order equals the
            // reference's sequential one. Otherwise replay it sequentially.
            double den;
            int ex = 0;
            if (!b && s > 0.0 && !__builtin_isinf(s)) ex = static_cast<int>((d2u(s) >> 52) & 0x7ffu) - 1023;
            if (!b && s > 0.0 && !__builtin_isinf(s) && mn >= ex - 51) {
                den = s;
            } else {
                den = 0.0;
                for (uint32_t i = 0; i < keff; ++i) den += static_cast<double>(prob[i]);
            }
            sh.f64[0] = den;
        }
        __syncthreads();
        const float inv_denom = static_cast<float>(1.0 / sh.f64[0]);
        int nan_p = 0;
        for (uint32_t i = tid; i < keff; i += kBlock) {
            const float pr = prob[i] * inv_denom;
            prob[i] = pr;
            if (__builtin_isnan(pr)) nan_p = 1;
        }
        nan_p = __any(nan_p);
        if (lane == 0) sh.i32[wave] = nan_p;
        __syncthreads();
        any_nan = (sh.i32[0] | sh.i32[1] | sh.i32[2] | sh.i32[3]) != 0;
        if (wave != 0) return;
    }
    // Wave 0: generation.cpp:103-126.
    auto seg_prob = [&](uint32_t g) {
        if (one_wave) return g == 0 ? pr_reg : 0.0f;
        const uint32_t i = g * 64 + static_cast<uint32_t>(lane);
        return i < keff ? prob[i] : 0.0f;
    };
    uint32_t pos;
    bool near;
    if (!any_nan && one_wave) scan_walk_wave(pr_reg, keff, p, u, prob, pos, near);
    else if (!any_nan) scan_and_walk_fast(seg_prob, prob, keff, p, u, pos, near);
    else scan_and_walk(seg_prob, keff, p, u, pos, near);
    const float ppos = one_wave ? readlane_f(pr_reg, static_cast<int>(pos)) : prob[pos];
    if (lane == 0)
        write_row(a, row, static_cast<int32_t>(composite_index(top[pos])), ppos, near ? GE_FLAG_NEAR_BOUNDARY : 0);
}

// A rescan of chunk c with m = k for the merge's fallback.
// Lean merge for the common rows (LeanList::on: k <= 64, not greedy, no
// penalty below 1), level j1 only and without a softcap: the chunks
// published their entries' final keys and the capped value of their j1-th
// entry. Every wave loads the chunks' counts, j1-th entries and capped bounds
// and reduces the row bound G1 (the largest j1-th entry) and its capped value
// B in registers; every thread loads one entry slot (chunk, position < j1)
// with its final key. Each wave compacts its entries above G1 (every element
// outside them ends at or below B) into its LDS segment as final composite
// keys; after the first barrier every thread ranks one entry over all
// segments by counting and stores it and its expf term at its rank when
// below k; after the second the top k is certified (its k-th final value
// above B, so nothing outside can reach or tie it) and wave 0 runs the
// reference's normalisation, min-p / top-p and draw (generation.cpp:89-126).
// Returns false (block-uniform, nothing written) when the lists do not
// certify; the caller then runs the full merge, which reloads them.
template <typename T>
__device__ __forceinline__ bool merge_lean(const DevArgs& a, SelShared& sh, const RowCtx& rc,
                                           const ge_sample_params& p, uint32_t k, const LeanList& ll,
                                           uint32_t stride, float u, uint32_t ej, uint32_t ec) {
    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int wave = tid >> 6;
    const uint32_t cpr = static_cast<uint32_t>(a.cpr);
    const uint32_t j1 = ll.j1;
    const uint64_t* slot_row = a.slots + static_cast<int64_t>(rc.row) * kSlotWords;

    // 1. One round trip: per wave the chunks' headers (lane c: chunk c), per
    //    thread one entry slot (chunk t % cpr, position t / cpr < j1) with its
    //    chunk's count and its final key, and the expf table.
    //    The loads are unconditional (lanes and positions past the lists read
    //    the last chunk's header or entry, and their words are then dropped):
    //    a load under a lane mask is followed by a wait for every load in
    //    flight, which would make this three round trips.
    const bool hl = static_cast<uint32_t>(lane) < cpr;
    const uint32_t hbase = min(static_cast<uint32_t>(lane), cpr - 1u) * stride;
    //    Words whose high half is not used are loaded as their low 32 bits
    //    (little-endian): a 64-bit load with a dead half lets the compiler
    //    reuse that register, which needs a wait for the load first.
    auto lo32 = [&](uint32_t w) { return load_shared(reinterpret_cast<const uint32_t*>(&slot_row[w])); };
    const uint64_t hg0 = load_shared(&slot_row[hbase]);
    const uint32_t hc0 = lo32(hbase + 1u);
    const uint64_t hj0 = load_shared(&slot_row[hbase + 1u + j1]);
    const uint32_t hb0 = lo32(hbase + ll.bound);
    const bool es = ej < j1;
    const uint32_t ebase = ec * stride;
    const uint32_t ejc = min(ej, j1 - 1u);
    const uint64_t er0 = load_shared(&slot_row[ebase + 2u + ejc]);
    const uint32_t ef0 = lo32(ebase + ll.fin + ejc);
    const uint32_t en0 = lo32(ebase + 1u);
    const uint64_t et = exp2_table(static_cast<uint32_t>(tid) & 31u);
    const uint64_t hg = hl ? hg0 : 0ull;
    const uint32_t hc = hl ? hc0 : 0u;
    const uint64_t hj = hl ? hj0 : 0ull;
    const uint32_t hb = hl ? hb0 : 0u;
    const uint64_t er = es ? er0 : 0ull;
    const uint32_t ef = es ? ef0 : 0u;
    const uint32_t en = es ? en0 : 0u;
    const float inv_temp = 1.0f / p.temperature;
    if (tid < 32) sh.exp_tab[tid] = et;
    // 2. G1 and B: over the chunks that listed j1 or more (a chunk that
    //    listed fewer listed everything). A failed chunk needs the full merge.
    if (__any(hl && hg == kGuaranteeFailed)) return false;  // every wave alike
    const bool lv = hl && static_cast<uint32_t>(hc) >= j1;
    const uint64_t vj = lv ? hj : 0ull;
    const uint32_t ghi = wave::max_u32(static_cast<uint32_t>(vj >> 32));
    const uint32_t glo = wave::max_u32(static_cast<uint32_t>(vj >> 32) == ghi ? static_cast<uint32_t>(vj) : 0u);
    const uint64_t g1 = (static_cast<uint64_t>(ghi) << 32) | glo;
    const uint32_t bkey = wave::max_u32(lv ? static_cast<uint32_t>(hb) : 0u);
    // 3. The entries above G1, as final composite keys, into stage[0, n):
    //    each wave takes its range with one LDS atomic (the counter and the
    //    maximum were cleared before the ticket's barrier); the row's largest
    //    final key by an LDS atomic maximum.
    const bool in = es && ej < static_cast<uint32_t>(en) && er > g1;
    const uint32_t fk = static_cast<uint32_t>(ef);
    const uint64_t mk = __ballot(in);
    const uint32_t n_w = static_cast<uint32_t>(__popcll(mk));
    const uint32_t kmax = wave::max_u32(in ? fk : 0u);
    uint32_t base = 0u;
    if (lane == 0 && n_w != 0u) {
        base = atomicAdd(&sh.u32[kSegCount], n_w);
        atomicMax(&sh.u32[8], kmax);
    }
    base = wave::readlane(base, 0);
    if (in) sh.stage[base + lanes_below(mk)] = composite(fk, raw_entry_index(er));
    __syncthreads();
    // 4. Rank over stage[0, n); the top k and their expf terms by rank.
    const uint32_t n = sh.u32[kSegCount];
    if (n < k) return false;  // block-uniform
    const float maximum = key_value(sh.u32[8]);
    float* ex = reinterpret_cast<float*>(sh.list);
    if (static_cast<uint32_t>(tid) < n) {
        const uint64_t x = sh.stage[tid];
        const float t = expf_glibc_tab((key_value(composite_key(x)) - maximum) * inv_temp,
                                       [&](uint32_t i) { return sh.exp_tab[i]; });
        // Four independent carry chains; blocks of 8 keys by 16-byte
        // broadcast reads, the last block masked (words past n are stale).
        const ulonglong2* p2 = reinterpret_cast<const ulonglong2*>(sh.stage);
        uint32_t r0 = 0, r1 = 0, r2 = 0, r3 = 0;
        const uint32_t full = n / 8u;
        uint32_t j = 0;
        for (; j + 2u <= full; j += 2u) {
            const ulonglong2 q0 = p2[4 * j + 0], q1 = p2[4 * j + 1], q2 = p2[4 * j + 2], q3 = p2[4 * j + 3];
            const ulonglong2 q4 = p2[4 * j + 4], q5 = p2[4 * j + 5], q6 = p2[4 * j + 6], q7 = p2[4 * j + 7];
            r0 = add_greater4(r0, q0.x, q0.y, q1.x, q1.y, x);
            r1 = add_greater4(r1, q2.x, q2.y, q3.x, q3.y, x);
            r2 = add_greater4(r2, q4.x, q4.y, q5.x, q5.y, x);
            r3 = add_greater4(r3, q6.x, q6.y, q7.x, q7.y, x);
        }
        if (j < full) {
            const ulonglong2 q0 = p2[4 * j + 0], q1 = p2[4 * j + 1], q2 = p2[4 * j + 2], q3 = p2[4 * j + 3];
            r0 = add_greater4(r0, q0.x, q0.y, q1.x, q1.y, x);
            r1 = add_greater4(r1, q2.x, q2.y, q3.x, q3.y, x);
            ++j;
        }
        if (8u * j < n) {
            const uint32_t b = 8u * j;
            uint64_t q[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) q[i] = b + static_cast<uint32_t>(i) < n ? sh.stage[b + static_cast<uint32_t>(i)] : 0ull;
            r2 = add_greater4(r2, q[0], q[1], q[2], q[3], x);
            r3 = add_greater4(r3, q[4], q[5], q[6], q[7], x);
        }
        const uint32_t rk = (r0 + r1) + (r2 + r3);
        if (rk < k) {
            sh.top[rk] = x;
            ex[rk] = t;
        }
    }
    __syncthreads();
    // 5. Certified when the k-th final value is above B.
    if (!(composite_key(sh.top[k - 1u]) > bkey)) return false;  // block-uniform
    if (wave != 0) return true;
    // 6. generation.cpp:89-126 over the k terms (wave 0).
    const bool live = static_cast<uint32_t>(lane) < k;
    const float e = live ? ex[lane] : 0.0f;
    const bool bad = live && (!(e >= 0.0f) || __builtin_isinf(e));
    const int lsb = (live && e > 0.0f && !bad) ? lsb_exponent(e) : INT_MAX;
    const double s = wave_sum(static_cast<double>(e));
    const int mn = wave_min_i(lsb);
    const int ex2 = static_cast<int>((d2u(s) >> 52) & 0x7ffu) - 1023;
    double den;
    // Exact when every term is a multiple of 2^mn and the sum fits 53 bits
    // above it: any order then equals the sequential sum.
    if (!__any(bad) && s > 0.0 && !__builtin_isinf(s) && mn >= ex2 - 51) {
        den = s;
    } else {
        den = 0.0;
        for (uint32_t i = 0; i < k; ++i) den += static_cast<double>(readlane_f(e, static_cast<int>(i)));
    }
    const float inv_denom = static_cast<float>(1.0 / den);
    const float pr = e * inv_denom;
    float* scratch = ex + 64;  // 64 floats for the sequential chains
    uint32_t pos;
    bool near;
    if (!__any(live && __builtin_isnan(pr))) {
        scan_walk_wave(pr, k, p, u, scratch, pos, near);
    } else {
        scan_and_walk([&](uint32_t g) { return g == 0 ? pr : 0.0f; }, k, p, u, pos, near);
    }
    const float ppos = readlane_f(pr, static_cast<int>(pos));
    if (lane == 0)
        write_row(a, rc.row, static_cast<int32_t>(composite_index(sh.top[pos])), ppos,
                  near ? GE_FLAG_NEAR_BOUNDARY : 0);
    return true;
}

// Merge for final-order lists (LeanList::fs: k above 64, no penalty below 1).
// Each chunk listed its top m by raw order as final composite keys sorted by
// final value, with B_c(m) and B_c(j1), the capped values of its m-th and
// j1-th raw entries: every element it left out (or left out of its first j1)
// ends at or below them. With B the largest bound of a level, the listed
// entries above B are a prefix of every list and hold every element above B;
// a 16-way merge of those prefixes (pairwise merge-path levels, each thread a
// run of outputs after one co-rank search) sorts them, and the top k is
// certified when its k-th final value is above B. Level j1 first, then level
// m. Returns false (block-uniform, nothing written) when neither certifies or
// a chunk failed.
template <typename T>
__device__ __forceinline__ bool merge_fs(const DevArgs& a, SelShared& sh, const RowCtx& rc,
                                         const ge_sample_params& p, uint32_t k, const LeanList& ll,
                                         uint32_t stride, float u) {
    static_assert(offsetof(SelShared, top) == offsetof(SelShared, list) + kListCap * sizeof(uint64_t) &&
                      kListCap + kMaxTopK >= kSlotWords + 2,
                  "list and top form the merge's second buffer");
    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const uint32_t cpr = static_cast<uint32_t>(a.cpr);
    const uint32_t words = cpr * stride;  // <= kSlotWords
    const uint32_t j1 = ll.j1;
    const uint64_t* slot_row = a.slots + static_cast<int64_t>(rc.row) * kSlotWords;
    constexpr int kPer = kSlotWords / kBlock;

    // 1. One round trip: every slot word, mirrored into stage at its own
    //    position (list c at c * stride + 2); per wave the chunks' headers
    //    (lane c: chunk c); the expf table.
    uint64_t w[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const uint32_t g = static_cast<uint32_t>(i * kBlock + tid);
        w[i] = g < words ? load_shared(&slot_row[g]) : 0ull;
    }
    const bool hl = static_cast<uint32_t>(lane) < cpr;
    const uint32_t hbase = static_cast<uint32_t>(lane) * stride;
    const uint64_t hg = hl ? load_shared(&slot_row[hbase]) : 0ull;
    const uint64_t hc = hl ? load_shared(&slot_row[hbase + 1u]) : 0ull;
    const uint64_t h1 = hl ? load_shared(&slot_row[hbase + stride - 1u]) : 0ull;
    const uint64_t et = tid < 32 ? exp2_table(static_cast<uint32_t>(tid)) : 0ull;
    if (tid < 32) sh.exp_tab[tid] = et;
    auto mirror = [&]() {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const uint32_t g = static_cast<uint32_t>(i * kBlock + tid);
            if (g < words) sh.stage[g] = w[i];
        }
    };
    mirror();
    if (__any(hl && hg == kGuaranteeFailed)) return false;  // every wave alike
    // 2. The level bounds, in every wave: B(j1) over the chunks that listed
    //    j1 or more (the others listed everything), B(m) over all.
    const uint32_t cnt_c = hl ? static_cast<uint32_t>(hc) : 0u;
    const uint32_t b1 = wave::max_u32((hl && cnt_c >= j1) ? static_cast<uint32_t>(h1) : 0u);
    const uint32_t bm = wave::max_u32(hl ? static_cast<uint32_t>(hg) : 0u);
    uint32_t levels = 0;
    while ((1u << levels) < cpr) ++levels;
    for (int lv = 0; lv < 2; ++lv) {
        const uint32_t B = lv == 0 ? b1 : bm;
        if (lv == 1) {
            if (bm == b1) break;  // the same bound again
            __syncthreads();      // the first try's reads are done
            mirror();
        }
        __syncthreads();
        // Prefix of list c above B (lists are in final order, keys distinct).
        uint32_t s_c = 0;
        if (hl) {
            const uint64_t* lst = sh.stage + hbase + 2u;
            uint32_t lo = 0, hi = cnt_c;
            while (lo < hi) {
                const uint32_t mid = (lo + hi) >> 1;
                if (composite_key(lst[mid]) > B) lo = mid + 1;
                else hi = mid;
            }
            s_c = lo;
        }
        const uint32_t incl = wave::incl_add(s_c);
        const uint32_t n = wave::readlane(incl, 63);
        if (n < k) continue;  // block-uniform
        if (tid < 64 && hl) sh.cnt[lane] = incl - s_c;  // exclusive prefix
        if (tid == 0) sh.cnt[cpr] = n;
        __syncthreads();
        // 3. Pairwise merge levels; the merge of chunks [c0, c2) lands at
        //    c0 * stride + 2 of the other buffer.
        const uint64_t* src = sh.stage;
        uint64_t* dst = sh.list;
        const uint32_t q = (n + kBlock - 1u) / kBlock;
        for (uint32_t l = 0; l < levels; ++l) {
            const uint32_t G = 1u << l;
            const uint32_t nout = (cpr + 2u * G - 1u) / (2u * G);
            uint32_t g = static_cast<uint32_t>(tid) * q;
            const uint32_t gend = min(g + q, n);
            while (g < gend) {
                // the output list holding g: the largest i with start(i) <= g
                uint32_t lo = 0, hi = nout;
                while (hi - lo > 1u) {
                    const uint32_t mid = (lo + hi) >> 1;
                    if (sh.cnt[mid * 2u * G] <= g) lo = mid;
                    else hi = mid;
                }
                const uint32_t c0 = lo * 2u * G, c1 = min(c0 + G, cpr), c2 = min(c0 + 2u * G, cpr);
                const uint32_t base = sh.cnt[c0];
                const uint32_t lenA = sh.cnt[c1] - base, lenB = sh.cnt[c2] - sh.cnt[c1];
                const uint64_t* A = src + c0 * stride + 2u;
                const uint64_t* Bp = src + c1 * stride + 2u;
                uint64_t* out = dst + c0 * stride + 2u;
                uint32_t o = g - base;
                const uint32_t oend = min(gend - base, lenA + lenB);
                uint32_t ca = o > lenB ? o - lenB : 0u, cb = min(o, lenA);
                while (ca < cb) {  // co-rank: A's share of the first o outputs
                    const uint32_t mid = (ca + cb) >> 1;
                    if (A[mid] > Bp[o - mid - 1u]) ca = mid + 1u;
                    else cb = mid;
                }
                uint32_t ia = ca, ib = o - ca;
                uint64_t va = ia < lenA ? A[ia] : 0ull, vb = ib < lenB ? Bp[ib] : 0ull;
                for (; o < oend; ++o) {
                    if (va > vb) {
                        out[o] = va;
                        ++ia;
                        va = ia < lenA ? A[ia] : 0ull;
                    } else {
                        out[o] = vb;
                        ++ib;
                        vb = ib < lenB ? Bp[ib] : 0ull;
                    }
                }
                g = base + oend;
            }
            __syncthreads();
            const uint64_t* t = src;
            src = dst;
            dst = const_cast<uint64_t*>(t);
        }
        // 4. Certified when the k-th final value is above B.
        const uint64_t* top = src + 2;
        if (!(composite_key(top[k - 1u]) > B)) continue;  // block-uniform
        merge_finish<T>(a, sh, rc, p, false, k, u, 0.0f, top, reinterpret_cast<float*>(dst));
        return true;
    }
    return false;
}

// Merge fallback for final-order lists: the top k of every listed entry into
// sh.top[0, nt), and in sh.gam[c] a bound for chunk c as merge_all_lists
// leaves it (a final composite key no element the chunk left out exceeds).
__device__ __forceinline__ void merge_all_fs(const DevArgs& a, SelShared& sh, const RowCtx& rc, uint32_t k,
                                             uint32_t stride, uint32_t& nt) {
    const int tid = threadIdx.x;
    constexpr int kPer = kSlotWords / kBlock;
    uint64_t w[kPer];
    uint32_t wp[kPer], wc[kPer];
    load_slots(a, sh, rc.row, stride, w, wp, wc);
    __syncthreads();
    bool ent[kPer];
    uint32_t cnt = 0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        ent[i] = slot_entry(sh, wp[i], wc[i]);
        cnt += ent[i] ? 1u : 0u;
    }
    uint32_t n;
    uint32_t pos = block_excl_scan(cnt, n, sh);
#pragma unroll
    for (int i = 0; i < kPer; ++i)
        if (ent[i]) sh.stage[pos++] = w[i];
    __syncthreads();
    for (int c = tid; c < a.cpr; c += kBlock) {
        const uint64_t g = sh.gam[c];
        if (g != 0ull && g != kGuaranteeFailed) sh.gam[c] = (g << 32) | 0xffffffffull;
    }
    __syncthreads();
    nt = select_top(sh.stage, n, k, sh.top);
}

template <typename T, int EPT, int SBE = 0>
__device__ __forceinline__ uint32_t rescan_chunk(const RowCtx& rc, int c, uint32_t k, uint32_t* pbits,
                                                 SelShared& sh, bool& ok) {
    uint32_t n_out;
    (void)chunk_slow<T, EPT, SBE>(rc, c * (kBlock * EPT), k, pbits, sh, n_out, ok);
    return n_out;
}

// Four waves per SIMD (at most 128 VGPRs): with 4 workgroups per CU, the
// 1024 workgroups of a 64-row batch are all resident from the start.
template <typename T, int EPT>
__global__ __launch_bounds__(kBlock, 4) void select_kernel(DevArgs a) {
    constexpr int CHUNK = kBlock * EPT;
    __shared__ uint32_t s_pbits[CHUNK / 32];
    __shared__ SelShared sh;

    const int tid = threadIdx.x;
    // Workgroups are dispatched to the 8 XCDs round-robin (block b to XCD
    // b % 8). When the rows split evenly, XCD x takes whole rows: the row's
    // lists then meet in one XCD's L2.
    int bid = static_cast<int>(blockIdx.x);
    if ((a.rows & 7) == 0) bid = (bid & 7) * static_cast<int>(gridDim.x >> 3) + (bid >> 3);
    const int row = bid / a.cpr;
    const int chunk = bid - row * a.cpr;
    const int V = a.vocab;
    const ge_sample_params p = row_params(a, row);
    const bool greedy = p.temperature <= 0.0f;  // generation.cpp:66
    const uint32_t k = greedy ? 1u
                              : (p.top_k ? min(p.top_k, static_cast<uint32_t>(V))
                                         : static_cast<uint32_t>(V));  // generation.cpp:80
    if (k > static_cast<uint32_t>(kMaxTopK)) {
        // The full-order kernels serve these rows; the host launches them
        // whenever the handle has their workspace.
        if (a.fo_items) return;
        if (chunk == 0 && tid == 0) {
            if (row_done(a, row)) {
                skipped_row(a, row);
            } else {
                a.tokens[row] = -1;
                if (a.probs) a.probs[row] = 0.0f;
                if (a.flags) a.flags[row] = GE_FLAG_UNSUPPORTED;
            }
        }
        return;
    }
    if (row_done(a, row)) {
        // Finished by an earlier call: nothing is read, no ticket is taken.
        if (chunk == 0 && tid == 0) skipped_row(a, row);
        return;
    }
    RowCtx rc;
    rc.rowp = static_cast<const T*>(a.logits) + static_cast<int64_t>(row) * a.row_stride;
    row_history(a, row, rc.hist, rc.H);
    rc.row = row;
    rc.V = V;
    rc.vec_ok = a.vec_ok;
    rc.r = p.repetition_penalty;
    rc.pen = rc.H > 0 && !(rc.r == 1.0f);
    rc.cap = p.softcap;
    const uint32_t m = spec_m(k, a.cpr, CHUNK);
    // Slot stride: room for about twice the usual candidate count (words
    // past a chunk's count are not read); with a penalty below 1 the row's
    // slot area split evenly, so a chunk can append its penalised tokens.
    const bool pen_all = rc.pen && !(rc.r >= 1.0f);
    const uint32_t stride = pen_all ? static_cast<uint32_t>(kSlotWords / a.cpr)
                                    : min(static_cast<uint32_t>(kSlotWords / a.cpr), 2u * m + 24u);
    uint64_t* slot = a.slots + static_cast<int64_t>(row) * kSlotWords + static_cast<int64_t>(chunk) * stride;

    // Lean rows (merge_lean): small k, no penalty below 1, every chunk's
    // first j1 entries within one word per thread; the chunks also publish
    // their entries' final keys.
    LeanList ll;
    ll.j1 = spec_level1(k, a.cpr, m);
    ll.cap = (stride - 3u) / 2u;
    ll.fin = 2u + ll.cap;
    ll.bound = 2u + 2u * ll.cap;
    ll.on = !greedy && k <= 64u && !pen_all && a.cpr <= 64 && m <= ll.cap &&
            static_cast<uint32_t>(a.cpr) * ll.j1 <= static_cast<uint32_t>(kBlock);
    ll.fs = !greedy && !ll.on && k > 64u && !pen_all && a.cpr <= 64 && m + 3u <= stride &&
            m <= static_cast<uint32_t>(kBlock);
    // The entry slot this thread loads if its workgroup merges (chunk
    // tid % cpr, position tid / cpr): the division runs while the logits load.
    const uint32_t lean_j = static_cast<uint32_t>(tid) / static_cast<uint32_t>(a.cpr);
    const uint32_t lean_c = static_cast<uint32_t>(tid) - lean_j * static_cast<uint32_t>(a.cpr);

    uint32_t n_top, n_out;
    bool direct, ok;
    const uint64_t gamma =
        chunk_topm<T, EPT>(rc, chunk * CHUNK, m, s_pbits, sh, slot, stride, ll, n_top, n_out, direct, ok);

    // Publish [guarantee, count, sorted entries] (a list ranked by one wave
    // or with appended penalised entries is already written), wait for the
    // stores, then one ticket per workgroup; the last workgroup of the row
    // merges.
    if (ll.fs) {
        if (direct) {
            __syncthreads();  // the list is written, the bounds are in sh.u32[24], [25]
        } else {
            // The list's final composite keys, ranked by final value; the capped
            // values of the m-th and j1-th raw entries as the bounds.
            const uint32_t i = static_cast<uint32_t>(tid);
            uint64_t fc = 0ull;
            if (i < n_top) {
                const uint64_t e = sh.list[i];
                const float f = softcap(key_value(static_cast<uint32_t>(e >> 32)), rc.cap);
                const uint32_t kc = order_key(f);
                fc = composite(order_key((rc.pen && raw_entry_pen(e)) ? penalize(f, rc.r) : f), raw_entry_index(e));
                if (i == m - 1u) sh.u32[24] = kc;
                if (i == ll.j1 - 1u) sh.u32[25] = kc;
            }
            sh.stage[i] = fc;  // zeros past n_top pad the rank's reads
            __syncthreads();
            if (i < n_top) {
                const ulonglong2* p2 = reinterpret_cast<const ulonglong2*>(sh.stage);
                uint32_t r0 = 0, r1 = 0;
                for (uint32_t j = 0; j < (n_top + 7u) / 8u; ++j) {
                    const ulonglong2 q0 = p2[4 * j + 0], q1 = p2[4 * j + 1], q2 = p2[4 * j + 2], q3 = p2[4 * j + 3];
                    r0 = add_greater4(r0, q0.x, q0.y, q1.x, q1.y, fc);
                    r1 = add_greater4(r1, q2.x, q2.y, q3.x, q3.y, fc);
                }
                store_shared(&slot[2u + r0 + r1], fc);
            }
        }
        if (tid == 0) {
            const uint64_t g0 = gamma == kGuaranteeFailed ? kGuaranteeFailed
                                                          : (gamma == 0ull ? 0ull : static_cast<uint64_t>(sh.u32[24]));
            store_shared(&slot[0], g0);
            store_shared(&slot[1], static_cast<uint64_t>(n_top));
            store_shared(&slot[stride - 1u], static_cast<uint64_t>(n_top >= ll.j1 ? sh.u32[25] : 0u));
        }
    } else if (tid == 0) {
        store_shared(&slot[0], gamma);
        store_shared(&slot[1], static_cast<uint64_t>(min(n_out, ll.on ? ll.cap : stride - 2u)));
    }
    if (!direct && !ll.fs) {
        for (uint32_t i = tid; i < n_top; i += kBlock) {
            const uint64_t e = sh.list[i];
            store_shared(&slot[2u + i], e);
            if (ll.on) {
                const float f = softcap(key_value(static_cast<uint32_t>(e >> 32)), rc.cap);
                store_shared(&slot[ll.fin + i],
                             static_cast<uint64_t>(order_key((rc.pen && raw_entry_pen(e)) ? penalize(f, rc.r) : f)));
                if (i == ll.j1 - 1u) store_shared(&slot[ll.bound], static_cast<uint64_t>(order_key(f)));
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        const uint32_t ticket =
            __hip_atomic_fetch_add(&a.tickets[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sh.u32[0] = ticket == static_cast<uint32_t>(a.cpr - 1) ? 1u : 0u;
        sh.u32[kSegCount] = 0u;  // merge_lean's entry counter and maximum
        sh.u32[8] = 0u;
    }
    __syncthreads();
    if (sh.u32[0] == 0u) return;

    // Row inputs of the merge's last steps (scalar loads), loaded now so
    // their latency overlaps the collection.
    const float u = greedy ? 0.0f : a.uniforms[row];
    const float x0 = greedy ? load_one(static_cast<const T*>(rc.rowp), 0) : 0.0f;
    if (ll.on) {
        if (merge_lean<T>(a, sh, rc, p, k, ll, stride, u, lean_j, lean_c)) return;
        __syncthreads();  // not certified: the full merge below reloads the lists
    }
    if (ll.fs) {
        if (merge_fs<T>(a, sh, rc, p, k, ll, stride, u)) return;
        // Not certified: every listed entry, then exact rescans.
        __syncthreads();
        uint32_t nt;
        merge_all_fs(a, sh, rc, k, stride, nt);
        for (int c = next_rescan(sh, 0, a.cpr, nt, k); c >= 0; c = next_rescan(sh, c + 1, a.cpr, nt, k)) {
            bool rok;
            const uint32_t nl = rescan_chunk<T, EPT>(rc, c, k, s_pbits, sh, rok);
            if (!rok) {
                if (tid == 0) write_row(a, row, -1, 0.0f, GE_FLAG_UNSUPPORTED);
                return;
            }
            nt = absorb_list(sh, nt, nl, k);
        }
        merge_finish<T>(a, sh, rc, p, false, min(nt, k), u, x0, sh.top, reinterpret_cast<float*>(sh.stage));
        return;
    }
    uint32_t nt;
    const bool collected = static_cast<uint32_t>(a.cpr) * stride <= static_cast<uint32_t>(kBlock * kSmallWords)
                               ? merge_collect_small(a, sh, rc, k, spec_level1(k, a.cpr, m), stride, nt)
                               : merge_collect(a, sh, rc, k, stride, nt);
    if (!collected) {
        // Fallback: every listed entry with its final value, then an exact
        // rescan of each chunk whose bound reaches the k-th largest so far.
        merge_all_lists(a, sh, rc, k, stride, nt);
        for (int c = next_rescan(sh, 0, a.cpr, nt, k); c >= 0; c = next_rescan(sh, c + 1, a.cpr, nt, k)) {
            bool rok;
            const uint32_t nl = rescan_chunk<T, EPT>(rc, c, k, s_pbits, sh, rok);
            if (!rok) {
                if (tid == 0) write_row(a, row, -1, 0.0f, GE_FLAG_UNSUPPORTED);
                return;
            }
            nt = absorb_list(sh, nt, nl, k);
        }
    }
    merge_finish<T>(a, sh, rc, p, greedy, min(nt, k), u, x0, sh.top, reinterpret_cast<float*>(sh.stage));
}

template <typename T, int EPT>
hipError_t launch_t(const DevArgs& a, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(a.rows * a.cpr));
    const dim3 block(kBlock);
    hipLaunchKernelGGL((select_kernel<T, EPT>), grid, block, 0, s, a);
    return hipGetLastError();
}

// ---- Single-pass selection with polled candidate lists (stream_kernel) -----
//
// For calls with shared parameters, 1 <= k <= 64, temperature > 0 and no
// penalty below 1 (CallPlan::run_stream), at 64 logits per thread and at most
// 16 chunks per row. The chunks publish unsorted candidate lists and leave; no
// chunk ranks anything, waits for its stores or takes a ticket at its end.
//
// Per chunk (workgroup), once its logits are in registers:
//   1. each wave takes the q_hi-th and q_lo-th largest of its 64 lane maxima;
//      the chunk's bounds tau_hi >= tau_lo are the smallest over its waves, so
//      at least 4 q elements of the chunk lie at or above each;
//   2. every wave lists the elements of its slots at or above tau_lo (a wave
//      with fewer than q_lo lane maxima lists all its non-NaN elements) as
//      final composite keys (softcap, then the penalty for history ids), and
//      publishes the capped values of tau_hi and tau_lo as its header.
// Every element a chunk leaves out has a raw value below tau_lo, so its final
// value is at most softcap(tau_lo) (softcap is monotone and a penalty >= 1
// never raises a value); with B the largest capped bound of the row at a
// level, every element whose final value exceeds B is listed. So when at
// least k listed entries exceed B, their top k (final value descending, index
// ascending) is the row's top k: everything outside ends at or below B.
//
// The merging workgroup of a row is its last chunk, the row's highest block
// index in dispatch order (also under the XCD-aware mapping): workgroups are
// dispatched in index order, so every other workgroup of the row has been
// dispatched before it, and they finish without waiting for anything; the
// merge's wait ends, resident grid or not. (A start ticket would pin this
// without the dispatch order, but its atomic's return, queued behind the
// streaming loads, held back every workgroup's loads: C2 30 us.) The wait is
// bounded all the same (kPlSpins: GE_FLAG_TIMEOUT). It polls the row's list
// words, which are zero between calls: a list is complete when its header and
// all its entry words are non-zero (each wave writes every word of its list,
// unused positions as kPlFiller). Then it clears them for the next call,
// takes the row's bound at level hi (or lo when hi leaves fewer than k
// entries), ranks the entries above it and runs the reference's softmax,
// min-p / top-p and draw (src/generation.cpp:89-126). A row with fewer than k
// entries above either bound, an overflowing list or a wait that runs out
// falls back to exact rescans of every chunk.
//
// Cross-workgroup words are agent-scope relaxed atomic stores and loads (the
// sc1 bit: coherent across the XCDs' L2s); each word is written once per call
// and read only after it is seen non-zero, and 64-bit aligned stores are
// single-copy atomic, so no fence or ordering between words is needed.

constexpr uint32_t kPlPer = 6;          // entry words per merging thread per list
constexpr uint32_t kPlMaxEntries = 62;  // entry positions of one list at most
constexpr uint64_t kPlFiller = 1;    // an unused entry position (value key 0: never a candidate)
constexpr uint64_t kPlOverflow = ~uint64_t{0}; // header of a list that could not hold its candidates
constexpr uint32_t kPlCand = 4;         // candidates a lane stages (more: the list overflows)
constexpr uint32_t kPlSpins = 1u << 22; // about 4 s of polling; every awaited workgroup has started

// Entry positions per list for a row of nl = 4 * cpr lists (nl <= 64). An
// area holds the nl headers, then each list's entries in turn: nl * (1 + ne)
// <= kPollListWords = kPlPer * kBlock words, so the merge reads the entries
// as kPlPer contiguous words per thread.
__device__ __forceinline__ uint32_t pl_entries(uint32_t nl) {
    return min(static_cast<uint32_t>(kPollListWords) / nl - 1u, kPlMaxEntries);
}

// Lane-maximum rank of the chunk bound for a row with effective top-k k over
// cpr chunks: with mu = k / cpr, about (mu + 2 sqrt(mu) + 4) / 4 per wave. Any
// value is correct (it only sets how many entries are listed); this one keeps
// the lists short while leaving at least k entries above the row's bound in
// nearly every row (simulated on the benchmark distributions).
// Deterministic, so every workgroup of a row agrees.
__device__ __forceinline__ uint32_t pl_rank(uint32_t k, int cpr, uint32_t entries) {
    const float mu = spec_mu(k, cpr);
    const uint32_t q = static_cast<uint32_t>(ceilf((mu + 2.0f * __builtin_amdgcn_sqrtf(mu) + 4.0f) * 0.25f));
    return min(max(q, 1u), max(min(16u, entries / 2u), 1u));
}

template <typename T, int EPT>
__global__ __launch_bounds__(kBlock, 4) void stream_kernel(DevArgs a) {
    constexpr int W = sizeof(T) == 4 ? 4 : 8;  // elements per 16-byte load
    constexpr int NV = EPT / W;                 // 16-byte loads per thread
    constexpr int NW = EPT * sizeof(T) / 4;     // 32-bit words per thread
    constexpr int CHUNK = kBlock * EPT;
    constexpr int NG = EPT / 4;                 // groups of 4 slots per thread
    static_assert(EPT % W == 0 && EPT <= 64 && EPT % 4 == 0, "bad tiling");
    __shared__ uint32_t s_pbits[CHUNK / 32];
    __shared__ SelShared sh;

    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int wave = tid >> 6;
    // XCD-aware mapping as in select_kernel: each XCD streams whole rows.
    int bid = static_cast<int>(blockIdx.x);
    if ((a.rows & 7) == 0) bid = (bid & 7) * static_cast<int>(gridDim.x >> 3) + (bid >> 3);
    const int row = bid / a.cpr;
    const int chunk = bid - row * a.cpr;
    const int V = a.vocab;
    const ge_sample_params p = a.params;  // launched only with shared parameters
    const uint32_t k = p.top_k ? min(p.top_k, static_cast<uint32_t>(V)) : static_cast<uint32_t>(V);  // generation.cpp:80
    if (row_done(a, row)) {
        // Finished by an earlier call: nothing is read, no ticket is taken.
        if (chunk == 0 && tid == 0) skipped_row(a, row);
        return;
    }
    RowCtx rc;
    rc.rowp = static_cast<const T*>(a.logits) + static_cast<int64_t>(row) * a.row_stride;
    row_history(a, row, rc.hist, rc.H);
    rc.row = row;
    rc.V = V;
    rc.vec_ok = a.vec_ok;
    rc.r = p.repetition_penalty;
    rc.pen = rc.H > 0 && !(rc.r == 1.0f);
    rc.cap = p.softcap;
    const T* rowp = static_cast<const T*>(rc.rowp);
    const int c0 = chunk * CHUNK;
    const int cend = min(c0 + CHUNK, V);
    const uint32_t nl = 4u * static_cast<uint32_t>(a.cpr);
    const uint32_t ne = pl_entries(nl);  // entry positions per list
    // The row's call count: its parity picks this call's list area.
    uint64_t* const prow_base = a.plists + static_cast<int64_t>(row) * kPollRowWords;
    const uint64_t epoch = scalar_load(prow_base + kPollEpochWord);
    uint64_t* const prow = prow_base + (epoch & 1ull) * kPollListWords;
    uint64_t* const pnext = prow_base + ((epoch + 1ull) & 1ull) * kPollListWords;

    // 1. The first kBlock * kLoadBatch history ids, then the chunk's 16-byte
    //    nontemporal loads; the chunk's penalty bitmap is built from the ids
    //    while the logits are in flight (as in chunk_topm).
    int hid[kLoadBatch];
    if (rc.pen) {
#pragma unroll
        for (int u = 0; u < kLoadBatch; ++u) hid[u] = rc.hist[min(u * kBlock + tid, rc.H - 1)];
    }
    auto mark_history = [&]() {
        if (!rc.pen) return;
        for (int w = tid; w < CHUNK / 32; w += kBlock) s_pbits[w] = 0u;
        __syncthreads();
        for (int base = 0; base < rc.H; base += kBlock * kLoadBatch) {
            if (base > 0) {
#pragma unroll
                for (int u = 0; u < kLoadBatch; ++u) hid[u] = rc.hist[min(base + u * kBlock + tid, rc.H - 1)];
            }
#pragma unroll
            for (int u = 0; u < kLoadBatch; ++u)
                if (base + u * kBlock + tid < rc.H && hid[u] >= c0 && hid[u] < cend)
                    atomicOr(&s_pbits[(hid[u] - c0) >> 5], 1u << ((hid[u] - c0) & 31));
        }
    };
    uint32_t d[NW];
    auto value = [&](int s) -> float {
        if constexpr (W == 4) return u2f(d[s]);
        else return u2f((s % 2 == 0) ? (d[s / 2] << 16) : (d[s / 2] & 0xffff0000u));
    };
    constexpr uint32_t kHole = 0x7fc00000u;  // NaN in out-of-range slots
    if (rc.vec_ok && c0 + CHUNK <= V) {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const u32x4 q = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rowp + c0 + (v * kBlock + tid) * W));
            d[4 * v + 0] = q.x;
            d[4 * v + 1] = q.y;
            d[4 * v + 2] = q.z;
            d[4 * v + 3] = q.w;
        }
        mark_history();
    } else {
        mark_history();
#pragma unroll
        for (int s = 0; s < EPT; ++s) {
            const int e = c0 + ((s / W) * kBlock + tid) * W + (s % W);
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
    const float u = a.uniforms[row];
    if (tid < 32) sh.exp_tab[tid] = exp2_table(static_cast<uint32_t>(tid));

    // 2. Maxima of groups of 4 slots and of the lane (fmaxf skips NaN).
    float gm[NG];
    float lmf = NAN;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        float x = value(g * 4);
#pragma unroll
        for (int j = 1; j < 4; ++j) x = fmaxf(x, value(g * 4 + j));
        gm[g] = x;
        lmf = fmaxf(lmf, x);
    }
    // bf16: the packed words made opaque, so that the unpacked floats are
    // recomputed in the staging loop instead of held in registers.
    if constexpr (W == 8) {
#pragma unroll
        for (int i = 0; i < NW; ++i) asm volatile("" : "+v"(d[i]));
    }
    // 3. The wave's q-th largest lane maximum (lanes whose maximum is NaN or
    //    -inf count as 0); 0 means fewer such lanes: no bound from this wave.
    //    (-inf is no bound: a row masked with -inf would otherwise list
    //    every masked element and overflow.)
    const uint32_t qlo = pl_rank(k, a.cpr, ne);
    uint32_t key = order_key(lmf);
    key = key > kKeyNegInf ? key : 0u;
    uint32_t tlo = 0u;
    for (uint32_t i = 0; i < qlo; ++i) {
        const uint32_t mx = wave::max_u32(key);
        const uint64_t eq = __ballot(key == mx);
        if (lane == __ffsll(static_cast<unsigned long long>(eq)) - 1) key = 0u;
        tlo = mx;
    }
    if (lane == 0) sh.u32[12 + wave] = tlo ? tlo : 0xffffffffu;
    __syncthreads();  // (also orders the bitmap's marks before the reads below)
    const uint32_t tau_lo = min(min(sh.u32[12], sh.u32[13]), min(sh.u32[14], sh.u32[15]));
    const bool merger = chunk == a.cpr - 1;

    // 4. Stage this wave's candidates: lane l keeps its c-th at seg[64 c + l]
    //    (c < kPlCand), then they move to cmp[0, n_w) in (c, lane) order. A
    //    group of 4 slots is examined only when some lane's group maximum
    //    reaches the bound; inside, every slot's word is written, to the
    //    lane's next candidate position or to its own dummy word: no branch
    //    per slot.
    // A wave without a bound of its own lists every element above -inf.
    const float floor_v = tlo ? key_value(tau_lo) : -FLT_MAX;
    uint64_t* seg = sh.stage + wave * kSeg;
    uint64_t* cmp = seg + kPlCand * 64;            // compacted candidates (at most kPlMaxEntries)
    constexpr uint32_t kDummy = kSeg - 64;          // per-lane dummy words
    static_assert(kPlCand * 64 + kPlMaxEntries <= kDummy, "staging layout");
    const uint32_t ebase = static_cast<uint32_t>(c0 + tid * W);
    uint32_t cnt = 0;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        if (__ballot(gm[g] >= floor_v) == 0ull) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int s = 4 * g + j;
            const float x = value(s);
            const bool c = x >= floor_v;
            const uint32_t e = ebase + static_cast<uint32_t>((s / W) * kBlock * W + s % W);
            const uint32_t slot = (c && cnt < kPlCand) ? 64u * cnt + static_cast<uint32_t>(lane)
                                                       : kDummy + static_cast<uint32_t>(lane);
            seg[slot] = (static_cast<uint64_t>(f2u(x)) << 32) | e;
            cnt += c ? 1u : 0u;
        }
    }
    const uint64_t m0 = __ballot(cnt > 0u), m1 = __ballot(cnt > 1u), m2 = __ballot(cnt > 2u), m3 = __ballot(cnt > 3u);
    const uint32_t p0 = static_cast<uint32_t>(__popcll(m0)), p1 = static_cast<uint32_t>(__popcll(m1));
    const uint32_t p2 = static_cast<uint32_t>(__popcll(m2)), p3 = static_cast<uint32_t>(__popcll(m3));
    const uint32_t n_w = p0 + p1 + p2 + p3;
    const bool overflow = __ballot(cnt > kPlCand) != 0ull || n_w > ne;
    if (!overflow) {
        uint64_t y0 = 0, y1 = 0, y2 = 0, y3 = 0;
        if (cnt > 0u) y0 = seg[lane];
        if (cnt > 1u) y1 = seg[64 + lane];
        if (cnt > 2u) y2 = seg[128 + lane];
        if (cnt > 3u) y3 = seg[192 + lane];
        if (cnt > 0u) cmp[lanes_below(m0)] = y0;
        if (cnt > 1u) cmp[p0 + lanes_below(m1)] = y1;
        if (cnt > 2u) cmp[p0 + p1 + lanes_below(m2)] = y2;
        if (cnt > 3u) cmp[p0 + p1 + p2 + lanes_below(m3)] = y3;
    }
    wave_lds_sync();
    // 5. Final keys (one softcap round for the wave: lane i < n_w takes
    //    candidate i, lane 63 the value of tau), then the list: entries,
    //    fillers, and the header [largest final key | capped tau]. With no
    //    bound in any wave, every element above -inf is listed and the
    //    bound is the capped -inf (NaN and -inf are what is left out).
    float xv = 0.0f;
    uint32_t idx = 0u;
    bool pen = false;
    const bool cand = !overflow && static_cast<uint32_t>(lane) < n_w;
    if (cand) {
        const uint64_t y = cmp[lane];
        xv = u2f(static_cast<uint32_t>(y >> 32));
        idx = static_cast<uint32_t>(y);
        if (rc.pen) {
            const uint32_t off = idx - static_cast<uint32_t>(c0);
            pen = ((s_pbits[off >> 5] >> (off & 31)) & 1u) != 0u;
        }
    } else if (lane == 63) {
        xv = tau_lo != 0xffffffffu ? key_value(tau_lo) : -INFINITY;
    }
    float f = softcap(xv, rc.cap);
    if (pen) f = penalize(f, rc.r);
    const uint32_t fk = order_key(f);
    const uint32_t wmax = wave::max_u32(cand ? fk : 0u);
    const uint32_t blo = wave::readlane(fk, 63);
    const uint64_t hword = overflow ? kPlOverflow : ((static_cast<uint64_t>(wmax) << 32) | blo);
    const uint64_t eword = cand ? composite(fk, idx) : kPlFiller;
    const uint32_t lj_own = static_cast<uint32_t>(chunk) * 4u + static_cast<uint32_t>(wave);
    if (!merger) {
        // Publish the list (header, then entries), then clear this wave's
        // share of the row's other area (the next call's; no call reads it
        // now): every word of it.
        if (static_cast<uint32_t>(lane) < ne) store_shared(&prow[nl + lj_own * ne + static_cast<uint32_t>(lane)], eword);
        if (lane == 0) store_shared(&prow[lj_own], hword);
        const uint32_t lanes = static_cast<uint32_t>(a.cpr - 1) * static_cast<uint32_t>(kBlock);
        for (uint32_t i = static_cast<uint32_t>(chunk) * kBlock + static_cast<uint32_t>(tid); i < kPollListWords; i += lanes)
            store_shared(&pnext[i], uint64_t{0});
        return;
    }
    // The merging chunk keeps its own four lists in LDS, laid out as in the
    // area (no global stores ahead of its polling loads: one wait counter
    // covers both): headers in own_h, entries contiguous in own_e.
    uint64_t* own_h = sh.list;
    uint64_t* own_e = sh.list + 4;
    if (static_cast<uint32_t>(lane) < ne) own_e[static_cast<uint32_t>(wave) * ne + static_cast<uint32_t>(lane)] = eword;
    if (lane == 0) own_h[wave] = hword;
    if (tid < 32) sh.hist[tid] = 0u;       // the merge's threshold histogram
    if (tid == 0) sh.u32[kSegCount] = 0u;  // and its entry counter
    __syncthreads();

    // ---- Merge (the row's last chunk) ----
    // 6. Poll: thread t reads header t % nl (each wave thus holds all nl) and
    //    the entry words t + kBlock i of the area, contiguous across lanes.
    //    The last four lists are this chunk's own, read from LDS. A list is
    //    complete when all its words are non-zero.
    const uint32_t lj = static_cast<uint32_t>(tid) % nl;
    const uint32_t nent = nl * ne;
    const uint32_t own0 = (nl - 4u) * ne;  // first entry word of the own lists
    uint32_t eidx[kPlPer];
    bool ev[kPlPer];
#pragma unroll
    for (uint32_t i = 0; i < kPlPer; ++i) {
        const uint32_t u = static_cast<uint32_t>(tid) + kBlock * i;
        ev[i] = u < nent;
        eidx[i] = min(u, nent - 1u);
    }
    const bool hmine = lj >= nl - 4u;
    uint64_t h = 0ull;
    uint64_t e[kPlPer];
    bool timed_out = true;
    for (uint32_t it = 0; it < kPlSpins; ++it) {
        // Unconditional loads (clamped positions): a load under a lane mask
        // is followed by a wait for every load in flight.
        h = load_shared(&prow[lj]);
#pragma unroll
        for (uint32_t i = 0; i < kPlPer; ++i) e[i] = load_shared(&prow[nl + eidx[i]]);
        if (hmine) h = own_h[lj - (nl - 4u)];
#pragma unroll
        for (uint32_t i = 0; i < kPlPer; ++i)
            if (eidx[i] >= own0) e[i] = own_e[eidx[i] - own0];
        bool ok = h != 0ull;
#pragma unroll
        for (uint32_t i = 0; i < kPlPer; ++i) ok = ok && (!ev[i] || e[i] != 0ull);
        const uint32_t flag = 20u + 4u * (it & 1u);  // alternate words: one barrier per round
        const bool missing = __ballot(!ok) != 0ull;   // (every lane votes: outside the lane-0 branch)
        if (lane == 0) sh.u32[flag + wave] = missing ? 1u : 0u;
        __syncthreads();
        if ((sh.u32[flag] | sh.u32[flag + 1] | sh.u32[flag + 2] | sh.u32[flag + 3]) == 0u) {
            timed_out = false;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    // 7. The next call on this row takes the other area (which the other
    //    chunks have cleared): the count goes up once, after the merge (every
    //    chunk of the row has read it by now, having published its list).
    auto bump_epoch = [&]() {
        if (tid == 0) store_shared(prow_base + kPollEpochWord, static_cast<uint64_t>(epoch + 1u));
    };

    // 8. The row's bound B (the largest capped bound) and largest final key
    //    kmax, from the headers every wave holds. The entries above B go to
    //    a 32-bin histogram of (kmax - key) >> sh: bins 0..j hold exactly the
    //    entries above kmax - (j + 1) << sh, so the first bin whose running
    //    count reaches k sets the smallest certified threshold on this grid
    //    (any threshold at or above B is valid), and only about k entries
    //    are ranked instead of every entry above B.
    const uint32_t bnd = wave::max_u32(static_cast<uint32_t>(h));
    const uint32_t kmax = wave::max_u32(static_cast<uint32_t>(h >> 32));
    const uint32_t span = kmax > bnd ? kmax - bnd - 1u : 0u;
    const int bsh = max(32 - __clz(static_cast<int>(span)) - 5, 0);
#pragma unroll
    for (uint32_t i = 0; i < kPlPer; ++i) {
        const uint32_t ky = static_cast<uint32_t>(e[i] >> 32);
        if (ev[i] && ky > bnd) atomicAdd(&sh.hist[(kmax - ky) >> bsh], 1u);
    }
    __syncthreads();
    const uint32_t hb = lane < 32 ? sh.hist[lane] : 0u;
    const uint32_t cum = wave::incl_add(hb);
    const uint64_t reach = __ballot(lane < 32 && cum >= k);
    const int jsel = reach ? __ffsll(static_cast<unsigned long long>(reach)) - 1 : 32;
    const uint32_t n = reach ? wave::readlane(cum, jsel) : 0u;
    if (!timed_out && kmax > bnd && n >= k && n <= static_cast<uint32_t>(kBlock)) {
        // 9. The selected entries into stage[0, n): per-thread counts, a
        //    wave scan, one LDS counter per wave.
        uint32_t c = 0u;
        bool sel[kPlPer];
#pragma unroll
        for (uint32_t i = 0; i < kPlPer; ++i) {
            const uint32_t ky = static_cast<uint32_t>(e[i] >> 32);
            sel[i] = ev[i] && ky > bnd && ((kmax - ky) >> bsh) <= static_cast<uint32_t>(jsel);
            c += sel[i] ? 1u : 0u;
        }
        const uint32_t incl = wave::incl_add(c);
        uint32_t base = 0u;
        if (lane == 63 && incl != 0u) base = atomicAdd(&sh.u32[kSegCount], incl);
        uint32_t pos = wave::readlane(base, 63) + incl - c;
#pragma unroll
        for (uint32_t i = 0; i < kPlPer; ++i)
            if (sel[i]) sh.stage[pos++] = e[i];
        __syncthreads();
        // 10. Rank by counting; the top k and their expf terms by rank. Up to
        //     64 entries: wave 0 alone (one entry per lane), no barrier.
        const bool one_wave = n <= 64u;
        if (one_wave && wave != 0) {
            bump_epoch();
            return;
        }
        const float maximum = key_value(kmax);
        const float inv_temp = 1.0f / p.temperature;
        float* ex = reinterpret_cast<float*>(sh.list);
        if (static_cast<uint32_t>(tid) < n) {
            const uint64_t x = sh.stage[tid];
            const float t = expf_glibc_tab((key_value(composite_key(x)) - maximum) * inv_temp,
                                           [&](uint32_t i) { return sh.exp_tab[i]; });
            const ulonglong2* p2 = reinterpret_cast<const ulonglong2*>(sh.stage);
            uint32_t r0 = 0, r1 = 0, r2 = 0, r3 = 0;
            const uint32_t full = n / 8u;
            uint32_t j = 0;
            for (; j + 2u <= full; j += 2u) {
                const ulonglong2 q0 = p2[4 * j + 0], q1 = p2[4 * j + 1], q2 = p2[4 * j + 2], q3 = p2[4 * j + 3];
                const ulonglong2 q4 = p2[4 * j + 4], q5 = p2[4 * j + 5], q6 = p2[4 * j + 6], q7 = p2[4 * j + 7];
                r0 = add_greater4(r0, q0.x, q0.y, q1.x, q1.y, x);
                r1 = add_greater4(r1, q2.x, q2.y, q3.x, q3.y, x);
                r2 = add_greater4(r2, q4.x, q4.y, q5.x, q5.y, x);
                r3 = add_greater4(r3, q6.x, q6.y, q7.x, q7.y, x);
            }
            if (j < full) {
                const ulonglong2 q0 = p2[4 * j + 0], q1 = p2[4 * j + 1], q2 = p2[4 * j + 2], q3 = p2[4 * j + 3];
                r0 = add_greater4(r0, q0.x, q0.y, q1.x, q1.y, x);
                r1 = add_greater4(r1, q2.x, q2.y, q3.x, q3.y, x);
                ++j;
            }
            if (8u * j < n) {
                const uint32_t b = 8u * j;
                uint64_t q[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) q[i] = b + static_cast<uint32_t>(i) < n ? sh.stage[b + static_cast<uint32_t>(i)] : 0ull;
                r2 = add_greater4(r2, q[0], q[1], q[2], q[3], x);
                r3 = add_greater4(r3, q[4], q[5], q[6], q[7], x);
            }
            const uint32_t rk = (r0 + r1) + (r2 + r3);
            if (rk < k) {
                sh.top[rk] = x;
                ex[rk] = t;
            }
        }
        if (one_wave) {
            wave_lds_sync();
        } else {
            __syncthreads();
            if (wave != 0) {
                bump_epoch();
                return;
            }
        }
        // 11. generation.cpp:89-126 over the k terms (wave 0).
        const bool live = static_cast<uint32_t>(lane) < k;
        const float et = live ? ex[lane] : 0.0f;
        const bool bad = live && (!(et >= 0.0f) || __builtin_isinf(et));
        const int lsb = (live && et > 0.0f && !bad) ? lsb_exponent(et) : INT_MAX;
        const double s = wave_sum(static_cast<double>(et));
        const int mn = wave_min_i(lsb);
        const int ex2 = static_cast<int>((d2u(s) >> 52) & 0x7ffu) - 1023;
        double den;
        // Exact when every term is a multiple of 2^mn and the sum fits 53 bits
        // above it: any order then equals the sequential sum.
        if (!__any(bad) && s > 0.0 && !__builtin_isinf(s) && mn >= ex2 - 51) {
            den = s;
        } else {
            den = 0.0;
            for (uint32_t i = 0; i < k; ++i) den += static_cast<double>(readlane_f(et, static_cast<int>(i)));
        }
        const float inv_denom = static_cast<float>(1.0 / den);
        const float pr = et * inv_denom;
        float* scratch = ex + 64;  // 64 floats for the sequential chains
        uint32_t wpos;
        bool near;
        if (!__any(live && __builtin_isnan(pr))) {
            scan_walk_wave(pr, k, p, u, scratch, wpos, near);
        } else {
            scan_and_walk([&](uint32_t g) { return g == 0 ? pr : 0.0f; }, k, p, u, wpos, near);
        }
        const float ppos = readlane_f(pr, static_cast<int>(wpos));
        if (lane == 0)
            emit_row(a, row, static_cast<int32_t>(composite_index(sh.top[wpos])), ppos,
                     near ? GE_FLAG_NEAR_BOUNDARY : 0);
        bump_epoch();
        return;
    }
    bump_epoch();
    if (timed_out) {
        if (tid == 0) emit_row(a, row, -1, 0.0f, GE_FLAG_TIMEOUT);
        return;
    }
    // 12. Fallback (fewer than k entries above the bound, or an overflowing
    //     list). Every listed entry goes into the top k; then a chunk is
    //     rescanned exactly (chunk_slow stages at most 2k entries, within
    //     kStage) only when an element it left out could still enter: its
    //     bound word, (capped tau) << 32 | 0xffffffff (at least the composite
    //     key of any element it left out), is above the running k-th entry;
    //     a chunk with an overflowing list always is. absorb_list drops the
    //     entries a rescan finds again.
    __syncthreads();
    if (tid < a.cpr) sh.gam[tid] = 0ull;
    if (tid == 0) sh.u32[kSegCount] = 0u;
    __syncthreads();
    if (static_cast<uint32_t>(tid) < nl)  // thread t < nl holds header t
        lds_max_u64(&sh.gam[static_cast<uint32_t>(tid) / 4u],
                    h == kPlOverflow ? kPlOverflow : ((h << 32) | 0xffffffffull));
    lds_wait();
    {
        uint32_t c = 0u;
        bool keep[kPlPer];
#pragma unroll
        for (uint32_t i = 0; i < kPlPer; ++i) {
            keep[i] = ev[i] && e[i] != kPlFiller;
            c += keep[i] ? 1u : 0u;
        }
        const uint32_t incl = wave::incl_add(c);
        uint32_t base = 0u;
        if (lane == 63 && incl != 0u) base = atomicAdd(&sh.u32[kSegCount], incl);
        uint32_t pos = wave::readlane(base, 63) + incl - c;
#pragma unroll
        for (uint32_t i = 0; i < kPlPer; ++i)
            if (keep[i]) sh.stage[pos++] = e[i];
    }
    __syncthreads();
    uint32_t nt = select_top(sh.stage, sh.u32[kSegCount], k, sh.top);
    for (int c = 0; c < a.cpr; ++c) {
        const uint64_t kth = nt < k ? 0ull : sh.top[k - 1u];
        if (!(sh.gam[c] > kth)) continue;
        bool rok;
        const uint32_t nlist = rescan_chunk<T, EPT, kSlowBatchStream>(rc, c, k, s_pbits, sh, rok);
        if (!rok) {
            if (tid == 0) emit_row(a, row, -1, 0.0f, GE_FLAG_UNSUPPORTED);
            return;
        }
        nt = absorb_list(sh, nt, nlist, k);
    }
    merge_finish<T>(a, sh, rc, p, false, min(nt, k), u, 0.0f, sh.top, reinterpret_cast<float*>(sh.stage));
}

template <typename T>
hipError_t launch_stream_t(const DevArgs& a, hipStream_t s) {
    hipLaunchKernelGGL((stream_kernel<T, kMaxEpt>), dim3(static_cast<unsigned>(a.rows * a.cpr)), dim3(kBlock), 0, s, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_select(const DevArgs& a, hipStream_t stream, int ept) {
    if (a.dtype == GE_DTYPE_BF16)
        return ept == 16 ? launch_t<uint16_t, 16>(a, stream) : launch_t<uint16_t, 64>(a, stream);
    return ept == 16 ? launch_t<float, 16>(a, stream) : launch_t<float, 64>(a, stream);
}

hipError_t launch_stream(const DevArgs& a, hipStream_t stream) {
    return a.dtype == GE_DTYPE_BF16 ? launch_stream_t<uint16_t>(a, stream) : launch_stream_t<float>(a, stream);
}

}  // namespace ge
