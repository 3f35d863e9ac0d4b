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

#include <climits>

#include "chain_math.h"
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

enum : uint32_t { kMetaItems = 0, kMetaExtras = 1, kMetaNan = 2, kMetaStatus = 3 };
enum : uint32_t { kStatusOk = 0, kStatusTooManyPenalised = 1 };

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

// Histogram word and field of a bin: bins b and b + 32768 share a word.
__device__ __forceinline__ uint32_t bin_word(uint32_t bin) { return bin & (kWords - 1); }
__device__ __forceinline__ uint32_t bin_shift(uint32_t bin) { return (bin >> 15) << 4; }

// ---- small helpers ---------------------------------------------------------

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
__device__ __forceinline__ double rld(double v, int lane) {
    return __builtin_bit_cast(double, rl64(__builtin_bit_cast(uint64_t, v), lane));
}

__device__ __forceinline__ uint32_t wave_incl_u32(uint32_t v) {
    const int lane = __lane_id();
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t t = __shfl_up(v, d, 64);
        if (lane >= d) v += t;
    }
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
    if (n == 0 || d == 0) return 0;
    return d > kSat / n ? kSat : n * d;
}

// Block-wide exclusive scan of one u32 per thread; returns the total too.
// `scratch` holds kWaves entries. Contains barriers: every thread must call.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* scratch, uint32_t& total) {
    const int lane = __lane_id();
    const int wave = threadIdx.x >> 6;
    const uint32_t incl = wave_incl_u32(v);
    if (lane == 63) scratch[wave] = incl;
    __syncthreads();
    uint32_t before = 0;
    total = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const uint32_t x = scratch[w];
        if (w < wave) before += x;
        total += x;
    }
    __syncthreads();
    return before + incl - v;
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
    uint32_t off[kThreads];               // items before each thread's bins
    uint64_t mask[kThreads];              // each thread's non-empty, non-NaN bins
    uint32_t spill[kSpillCap];            // bins that moved 32768 counts out of LDS
    uint32_t scan[kWaves];
    uint32_t counters[4];                 // [0] penalised tokens, [1] spills, [2] NaN tokens
};

// Count of bin `bin` after streaming: the LDS field plus 32768 per spill.
__device__ __forceinline__ uint32_t bin_count(const HistShared& sh, uint32_t bin, uint32_t nspill) {
    uint32_t c = (sh.hist[bin_word(bin)] >> bin_shift(bin)) & 0xFFFFu;
    for (uint32_t i = 0; i < nspill; ++i) c += sh.spill[i] == bin ? 32768u : 0u;
    return c;
}

__global__ __launch_bounds__(kThreads) void fo_hist_kernel(DevArgs a) {
    __shared__ HistShared sh;
    const int tid = threadIdx.x;
    const int row = blockIdx.x;
    const int V = a.vocab;
    const ge_sample_params p = params_of(a, row);
    uint32_t k;
    if (!full_order_row(p, V, k)) return;

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
    uint32_t* meta = a.fo_meta + static_cast<int64_t>(row) * 4;
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

    auto count_token = [&](uint32_t bits16) {
        const uint32_t bin = bin_of(bits16);
        atomicAdd(&sh.hist[bin_word(bin)], 1u << bin_shift(bin));
    };
    auto penalised = [&](int idx) -> bool {
        return pen && ((bitmap[idx >> 5] >> (idx & 31)) & 1u);
    };
    const bool vec = a.vec_ok != 0;
    constexpr int kVecPerThread = kSubChunk / (kThreads * 8);  // 4 uint4 of 8 bf16
    for (int base = 0; base < V; base += kSubChunk) {
        if (vec && base + kSubChunk <= V) {
            uint4 q[kVecPerThread];
            uint32_t bm[kVecPerThread];
#pragma unroll
            for (int j = 0; j < kVecPerThread; ++j) {
                const int pos = base + (j * kThreads + tid) * 8;
                q[j] = *reinterpret_cast<const uint4*>(rowp + pos);
                bm[j] = pen ? (bitmap[pos >> 5] >> (pos & 31)) : 0u;
            }
#pragma unroll
            for (int j = 0; j < kVecPerThread; ++j) {
                const uint32_t w4[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
#pragma unroll
                for (int h = 0; h < 8; ++h) {
                    if ((bm[j] >> h) & 1u) continue;
                    count_token((w4[h >> 1] >> ((h & 1) * 16)) & 0xFFFFu);
                }
            }
        } else {
            for (int j = 0; j < kSubChunk / kThreads; ++j) {
                const int idx = base + j * kThreads + tid;
                if (idx < V && !penalised(idx)) count_token(rowp[idx]);
            }
        }
        __syncthreads();
        // Sweep: at most kSubChunk counts arrive between sweeps, so a field
        // below 32768 after a sweep cannot pass 65535 before the next one.
        for (uint32_t w = tid; w < kWords; w += kThreads) {
            const uint32_t x = sh.hist[w];
            uint32_t sub = 0;
            if ((x & 0xFFFFu) >= 0x8000u) {
                sub += 0x8000u;
                const uint32_t s = atomicAdd(&sh.counters[1], 1u);
                if (s < kSpillCap) sh.spill[s] = w;
            }
            if ((x >> 16) >= 0x8000u) {
                sub += 0x80000000u;
                const uint32_t s = atomicAdd(&sh.counters[1], 1u);
                if (s < kSpillCap) sh.spill[s] = w + kWords;
            }
            if (sub) sh.hist[w] = x - sub;
        }
        __syncthreads();
    }
    const uint32_t nspill = min(sh.counters[1], static_cast<uint32_t>(kSpillCap));

    // 3. Items in descending order. Thread t owns bins hb - j, j = 0..63,
    //    hb = 65535 - 64 t (bit j of its mask).
    const uint32_t hb = 65535u - 64u * static_cast<uint32_t>(tid);
    uint64_t mask = 0;
    uint32_t nan_local = 0;
    for (int j = 0; j < 64; ++j) {
        const uint32_t bin = hb - j;
        const uint32_t c = bin_count(sh, bin, nspill);
        if (c) {
            if (bin_is_nan(bin)) nan_local += c;
            else mask |= 1ull << j;
        }
    }
    uint32_t nbins_total;
    const uint32_t off = block_excl_scan(static_cast<uint32_t>(__popcll(mask)), sh.scan, nbins_total);
    sh.off[tid] = off;
    sh.mask[tid] = mask;
    if (nan_local) atomicAdd(&sh.counters[2], nan_local);
    __syncthreads();

    // Bin items: position = bins before + penalised tokens with a larger final value.
    {
        uint32_t c = 0;  // penalised tokens with thr_bin > bin (thr_bin is non-increasing)
        {
            uint32_t lo = 0, hi = E;
            while (lo < hi) {
                const uint32_t mid = (lo + hi) >> 1;
                if (sh.thr_bin[mid] > hb) lo = mid + 1;
                else hi = mid;
            }
            c = lo;
        }
        uint32_t rank = 0;
        for (int j = 0; j < 64; ++j) {
            if (!((mask >> j) & 1u)) continue;
            const uint32_t bin = hb - j;
            while (c < E && sh.thr_bin[c] > bin) ++c;
            const uint32_t cnt = bin_count(sh, bin, nspill);
            items[off + rank + c] = (static_cast<uint64_t>(f2u(bin_value(bin, cap))) << 32) | cnt;
            ++rank;
        }
    }
    // Penalised items: position = own rank + bins with a final value >= its own.
    for (uint32_t e = tid; e < E; e += kThreads) {
        const uint32_t tb = sh.thr_bin[e];
        uint32_t nb = 0;
        if (tb <= kHighBin) {
            const uint32_t t = (65535u - tb) >> 6;
            const uint32_t jt = (65535u - 64u * t) - tb;  // bit of bin tb in thread t's mask
            const uint64_t upto = jt == 63 ? ~0ull : ((2ull << jt) - 1);
            nb = sh.off[t] + static_cast<uint32_t>(__popcll(sh.mask[t] & upto));
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

// ---- kernel 2: probabilities, exact chains, token ----------------------------

struct ChainPos {
    int item;       // item holding the next (or the event) element
    uint32_t off;   // elements of that item before it
    uint32_t elem;  // global element index
};

// Replays elements [cp.elem, L) of the accumulation described by items
// (count in the low 32 bits) and per-item addends, with one wave. kDesc:
// c -= a, stopping at the first element with c <= a; else s += a, stopping
// at the first element whose sum is >= thr (NaN: never). On an event returns
// true with cp at the event element. Otherwise returns false with cp.elem == L
// and (cp.item, cp.off - 1) the last element consumed. Requires cp.elem < L.
template <typename Acc, bool kDesc>
__device__ bool wave_chain(const uint64_t* items, const float* add, int G, ChainPos& cp, uint32_t L,
                           double& s, double thr) {
    constexpr int P = chain::AccTraits<Acc>::P;
    const int lane = __lane_id();
    while (cp.elem < L && cp.item < G) {
        const int idx = cp.item + lane;
        uint32_t n = 0;
        double av = 0.0;
        if (idx < G) {
            n = static_cast<uint32_t>(items[idx]);
            av = static_cast<double>(add[idx]);
        }
        if (lane == 0) n -= cp.off;
        const uint32_t cincl = wave_incl_u32(n);
        const uint32_t cexcl = cincl - n;
        const uint32_t room = L - cp.elem;
        const uint32_t nt = cexcl >= room ? 0u : min(n, room - cexcl);
        const chain::Binade b = chain::binade_of<Acc>(s);
        const chain::Step st = chain::step_of<Acc>(b, av);
        const uint64_t tot = (nt && !st.big) ? sat_mul(nt, st.D) : 0;
        const uint64_t incl = wave_incl_u64_sat(tot);
        bool ev = false;
        if (nt) {
            if (kDesc) {
                // big: a reaches past c's binade, so c <= a and the walk stops here
                ev = st.big || st.tie || b.m < b.lo + incl;
            } else {
                uint64_t tm = chain::kNone;
                if (thr == thr) {
                    if (!(thr > 0.0)) tm = 0;
                    else if (thr < std::ldexp(1.0, b.uexp + P)) tm = chain::threshold_m(thr, b.uexp);
                }
                ev = st.big || st.tie || b.m + incl > b.hi || b.m + incl >= tm;
            }
        }
        const uint64_t evmask = __ballot(ev);
        if (evmask == 0) {
            const uint64_t total = rl64(incl, 63);
            const uint64_t m2 = kDesc ? b.m - total : b.m + total;
            s = std::ldexp(static_cast<double>(m2), b.uexp);
            const uint32_t all = rl32(cincl, 63);
            if (all >= room) {  // the last element lies in this tile
                const uint64_t lm = __ballot(n && cexcl < room && room <= cincl);
                const int l = static_cast<int>(__builtin_ctzll(lm));
                const uint32_t before = rl32(cexcl, l);
                cp.off = (l == 0 ? cp.off : 0u) + (room - before);
                cp.item += l;
                cp.elem = L;
                return false;
            }
            cp.elem += all;
            cp.item += 64;
            cp.off = 0;
            continue;
        }
        const int f = static_cast<int>(__builtin_ctzll(evmask));
        const uint64_t before = f ? rl64(incl, f - 1) : 0;
        const uint64_t m2 = kDesc ? b.m - before : b.m + before;
        s = std::ldexp(static_cast<double>(m2), b.uexp);
        cp.elem += rl32(cexcl, f);
        const uint32_t nf = rl32(nt, f);
        const double af = rld(av, f);
        const uint32_t offf = f == 0 ? cp.off : 0u;
        bool evt = false;
        const uint64_t used = kDesc ? chain::desc_run<Acc>(s, af, nf, evt)
                                    : chain::asc_run<Acc>(s, af, nf, thr, evt);
        cp.item += f;
        if (evt) {
            const uint32_t at = static_cast<uint32_t>(kDesc ? used : used - 1);
            cp.off = offf + at;
            cp.elem += at;
            return true;
        }
        cp.elem += nf;
        if (cp.elem >= L) {
            cp.off = offf + nf;
            return false;
        }
        cp.item += 1;
        cp.off = 0;
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

struct DecideShared {
    uint32_t gx_ids[kFoExtrasCap];  // penalised tokens of the selected value, ascending
    double dred[kWaves];
    int ired[kWaves];
    uint32_t ured[kWaves];
    uint32_t scan[kWaves];
    double den;
    float choice;
    uint32_t keep, pos, group_rank, group_total, forward, gx_count;
    uint32_t blo, bhi, nan_group, found;
    int32_t token;
    int item;
};

template <typename T, typename Op>
__device__ __forceinline__ T wave_reduce(T v, Op op) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v = op(v, __shfl_xor(v, d, 64));
    return v;
}

__global__ __launch_bounds__(kThreads) void fo_decide_kernel(DevArgs a) {
    __shared__ DecideShared sh;
    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int wave = tid >> 6;
    const int row = blockIdx.x;
    const int V = a.vocab;
    const ge_sample_params p = params_of(a, row);
    uint32_t k;
    if (!full_order_row(p, V, k)) return;

    const int32_t* hist;
    int H;
    history_of(a, row, hist, H);
    const bool pen = H > 0 && !(p.repetition_penalty == 1.0f);
    uint32_t* bitmap = a.fo_bitmap + static_cast<int64_t>(row) * a.fo_bitmap_words;
    const uint32_t* meta = a.fo_meta + static_cast<int64_t>(row) * 4;
    auto finish = [&](int32_t token, float prob, int32_t flags) {
        if (tid == 0) {
            a.tokens[row] = token;
            if (a.probs) a.probs[row] = prob;
            if (a.flags) a.flags[row] = flags;
            if (a.ring) {
                const uint32_t len = static_cast<uint32_t>(a.ring_len[row]);
                a.ring[static_cast<int64_t>(row) * a.ring_capacity +
                       static_cast<int64_t>(len % static_cast<uint32_t>(a.ring_capacity))] = token;
                a.ring_len[row] = static_cast<int32_t>(len + 1u);
            }
        }
        // The bitmap is all zero again after every call.
        if (pen) {
            __syncthreads();
            for (int i = tid; i < H; i += kThreads) {
                const int32_t id = hist[i];
                if (id >= 0 && id < V) bitmap[id >> 5] = 0u;
            }
        }
    };
    if (meta[kMetaStatus] != kStatusOk) {
        finish(-1, 0.0f, GE_FLAG_UNSUPPORTED);
        return;
    }
    const int G = static_cast<int>(meta[kMetaItems]);
    const uint64_t* items = a.fo_items + static_cast<int64_t>(row) * a.fo_items_stride;
    float* aux = a.fo_aux + static_cast<int64_t>(row) * a.fo_items_stride;
    uint32_t* pre = a.fo_pre + static_cast<int64_t>(row) * a.fo_items_stride;
    const uint64_t* extras = a.fo_extras + static_cast<int64_t>(row) * a.fo_extras_cap;
    const uint32_t E = meta[kMetaExtras];

    // 4a. Per item: elements before it, exp, certificate of the double sum.
    //     generation.cpp:94-97: p = exp((l - max) * (1/T)) in float.
    const float inv_temp = 1.0f / p.temperature;
    const float vmax = u2f(static_cast<uint32_t>(items[0] >> 32));
    const float p0 = expf_glibc((vmax - vmax) * inv_temp);
    const int per = (G + kThreads - 1) / kThreads;
    const int i_begin = min(G, tid * per);
    const int i_end = min(G, i_begin + per);
    uint32_t local = 0;
    for (int i = i_begin; i < i_end; ++i) local += static_cast<uint32_t>(items[i]);
    uint32_t total_elems;
    uint32_t run = block_excl_scan(local, sh.scan, total_elems);
    double S = 0.0;
    int minlsb = INT_MAX;
    bool nan = false;
    for (int i = i_begin; i < i_end; ++i) {
        const uint32_t n = static_cast<uint32_t>(items[i]);
        pre[i] = run;
        const uint32_t nk = run >= k ? 0u : min(n, k - run);
        run += n;
        const float v = u2f(static_cast<uint32_t>(items[i] >> 32));
        const float pe = expf_glibc((v - vmax) * inv_temp);
        aux[i] = pe;
        if (nk) {
            if (pe != pe) nan = true;
            else if (pe > 0.0f) {
                minlsb = min(minlsb, lsb_exp(pe));
                S += static_cast<double>(nk) * static_cast<double>(pe);
            }
        }
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
    if (tid == 0) {
        double St = 0.0;
        int ml = INT_MAX;
        uint32_t nn = 0;
        for (int w = 0; w < kWaves; ++w) {
            St += sh.dred[w];
            ml = min(ml, sh.ired[w]);
            nn |= sh.ured[w];
        }
        sh.dred[0] = St;
        sh.ired[0] = ml;
        sh.ured[0] = nn;
    }
    __syncthreads();
    const bool any_nan = sh.ured[0] != 0;
    // Every term is a multiple of 2^minlsb; if the sum needs at most 53 bits
    // above that, every partial sum in every order is exact, so the parallel
    // sum equals the reference's sequential one (generation.cpp:97).
    const double Sp = sh.dred[0];
    const bool certified = !any_nan && (Sp == 0.0 || sh.ired[0] >= exp_of(Sp) - 51);
    if (wave == 0) {
        double den = Sp;
        if (any_nan) {
            den = __builtin_nan("");
        } else if (!certified) {
            ChainPos cp{0, 1, 1};
            double s = static_cast<double>(p0);
            if (k > 1) wave_chain<double, false>(items, aux, G, cp, k, s, __builtin_nan(""));
            den = s;
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
    for (int i = i_begin; i < i_end; ++i) {
        const float q = aux[i] * inv;
        aux[i] = q;
        if (i >= 1 && pre[i] < k && q < minimum && first_low == INT_MAX) first_low = i;
    }
    first_low = wave_reduce(first_low, [](int x, int y) { return min(x, y); });
    if (lane == 0) sh.ired[wave] = first_low;
    __syncthreads();
    if (wave == 0) {
        int fl = lane < kWaves ? sh.ired[lane] : INT_MAX;
        fl = wave_reduce(fl, [](int x, int y) { return min(x, y); });
        // generation.cpp:106-115: min-p stops before element e >= 1 with p_e < minimum.
        uint32_t keff = k;
        if (!any_nan) {
            if (q0 < minimum) keff = 1;
            else if (fl != INT_MAX) keff = min(keff, pre[fl]);
        }
        uint32_t keep, pos;
        int item;
        float choice = __builtin_nanf("");
        bool near = false;
        if (any_nan) {
            // NaN probabilities: no cut fires and the walk never stops.
            keep = k;
            pos = k - 1;
            item = wave_find_item(pre, G, pos);
        } else {
            // generation.cpp:105-113: fp32 cumulative, top-p stop needs keep > 0.
            double s = static_cast<double>(q0);
            ChainPos cp{0, 1, 1};
            keep = keff;
            if (keff > 1 && wave_chain<float, false>(items, aux, G, cp, keff, s, static_cast<double>(p.top_p)))
                keep = cp.elem + 1;
            const float mass = static_cast<float>(s);
            // random.h:1864-1871 and generation.cpp:118-124.
            const float u = a.uniforms[row];
            choice = u * (mass - 0.0f) + 0.0f;
            if (choice > 0.0f && choice < __builtin_inff()) {
                ChainPos w{0, 0, 0};
                double c = static_cast<double>(choice);
                if (wave_chain<float, true>(items, aux, G, w, keep, c, 0.0)) {
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
            // before and through the chosen position (as the oracle defines it).
            double c_before = 0.0;
            if (pos > 0) {
                // exact parallel sum when certified, else the closed-form chain
                double sum = 0.0;
                int ml = INT_MAX;
                for (int i0 = 0; i0 <= item; i0 += 64) {
                    const int i = i0 + lane;
                    if (i <= item) {
                        const uint32_t n = static_cast<uint32_t>(items[i]);
                        const uint32_t pi = pre[i];
                        const uint32_t cnt = pi >= pos ? 0u : min(n, pos - pi);
                        const float q = aux[i];
                        if (cnt && q > 0.0f) {
                            sum += static_cast<double>(cnt) * static_cast<double>(q);
                            ml = min(ml, lsb_exp(q));
                        }
                    }
                }
                sum = wave_reduce(sum, [](double x, double y) { return x + y; });
                ml = wave_reduce(ml, [](int x, int y) { return min(x, y); });
                if (sum == 0.0 || ml >= exp_of(sum) - 51) {
                    c_before = sum;
                } else {
                    ChainPos cp2{0, 1, 1};
                    double sb = static_cast<double>(q0);
                    if (pos > 1) wave_chain<double, false>(items, aux, G, cp2, pos, sb, __builtin_nan(""));
                    c_before = sb;
                }
            }
            const double c_at = c_before + static_cast<double>(aux[item]);
            const double ch = static_cast<double>(choice);
            near = (pos > 0 && __builtin_fabs(ch - c_before) < 1e-6) ||
                   (pos + 1 < keep && __builtin_fabs(ch - c_at) < 1e-6);
        }
        if (lane == 0) {
            sh.keep = keep;
            sh.pos = pos;
            sh.item = item;
            sh.choice = choice;
            sh.found = near ? 1u : 0u;  // reused below; flag kept in a register copy
        }
    }
    __syncthreads();
    const uint32_t pos = sh.pos;
    const int item = sh.item;
    const bool near = sh.found != 0;
    __syncthreads();

    // 6. The selected value's group: items with the same order key are
    //    adjacent; its tokens are the bins with that key (not penalised) and
    //    the penalised tokens with that key.
    const float cap = p.softcap;
    if (wave == 0) {
        const uint32_t key = order_key(u2f(static_cast<uint32_t>(items[item] >> 32)));
        int is = item, ie = item;
        for (;;) {  // first item of the group
            const int i = is - 1 - lane;
            const bool same = i >= 0 && order_key(u2f(static_cast<uint32_t>(items[i] >> 32))) == key;
            const uint64_t m = __ballot(same);
            const int run_len = m == ~0ull ? 64 : static_cast<int>(__builtin_ctzll(~m));
            is -= run_len;
            if (run_len < 64) break;
        }
        for (;;) {  // last item of the group
            const int i = ie + 1 + lane;
            const bool same = i < G && order_key(u2f(static_cast<uint32_t>(items[i] >> 32))) == key;
            const uint64_t m = __ballot(same);
            const int run_len = m == ~0ull ? 64 : static_cast<int>(__builtin_ctzll(~m));
            ie += run_len;
            if (run_len < 64) break;
        }
        const uint32_t first = pre[is];
        const uint32_t total = pre[ie] + static_cast<uint32_t>(items[ie]) - first;
        const uint32_t rank = pos - first;
        // bins [blo, bhi] whose final value has this key (empty when blo > bhi)
        uint32_t blo = 1, bhi = 0;
        const bool nan_group = key == kKeyNaN;
        if (!nan_group) {
            // lower_bound of key, and of key + 1, over [kLowBin, kHighBin + 1)
            uint32_t bounds[2];
            for (int t = 0; t < 2; ++t) {
                const uint32_t want = key + static_cast<uint32_t>(t);
                uint32_t lo = kLowBin, hi = kHighBin + 1;  // first bin with bin_key >= want in [lo, hi]
                while (hi > lo) {
                    const uint32_t span = hi - lo;
                    const uint32_t step = (span + 63) / 64;
                    const uint32_t probe = lo + static_cast<uint32_t>(lane) * step;
                    const bool below = probe < hi && bin_key(probe, cap) < want;
                    const uint64_t m = __ballot(below);
                    if (m == 0) break;  // bin lo already >= want
                    const int last = 63 - static_cast<int>(__builtin_clzll(m));
                    lo = lo + static_cast<uint32_t>(last) * step + 1;
                    hi = min(hi, lo - 1 + step);
                }
                bounds[t] = lo;
            }
            blo = bounds[0];
            bhi = bounds[1] - 1;
        }
        // penalised tokens with this key: a contiguous run of the sorted extras
        uint32_t xs = 0, xe = 0;
        if (E > 0) {
            uint32_t b2[2];
            for (int t = 0; t < 2; ++t) {
                // first extra whose key is <= key - t... keys are descending:
                // count of extras with key > (key - 1 + t) ... computed as lower bounds
                const uint32_t want = key + 1u - static_cast<uint32_t>(t);  // t=0: > key, t=1: >= key
                uint32_t lo = 0, hi = E;  // first index with composite_key < want
                while (hi > lo) {
                    const uint32_t span = hi - lo;
                    const uint32_t step = (span + 63) / 64;
                    const uint32_t probe = lo + static_cast<uint32_t>(lane) * step;
                    const bool ge_want = probe < hi && composite_key(extras[probe]) >= want;
                    const uint64_t m = __ballot(ge_want);
                    if (m == 0) break;
                    const int last = 63 - static_cast<int>(__builtin_clzll(m));
                    lo = lo + static_cast<uint32_t>(last) * step + 1;
                    hi = min(hi, lo - 1 + step);
                }
                b2[t] = lo;
            }
            xs = b2[0];  // extras with key > this key come first
            xe = b2[1];  // ... then those equal to it
        }
        if (lane == 0) {
            sh.group_rank = rank;
            sh.group_total = total;
            sh.blo = blo;
            sh.bhi = bhi;
            sh.nan_group = nan_group ? 1u : 0u;
            sh.gx_count = xe - xs;
            sh.forward = (rank <= (total - 1) / 2) ? 1u : 0u;
            sh.found = 0;
            sh.token = -1;
        }
        for (uint32_t x = xs + static_cast<uint32_t>(lane); x < xe; x += 64)
            sh.gx_ids[x - xs] = composite_index(extras[x]);
    }
    __syncthreads();

    // Locate the token: the rank-th lowest index of the group (or the
    // (total-1-rank)-th highest), in batches of 8192 tokens from that end.
    {
        const bool fwd = sh.forward != 0;
        uint32_t want = fwd ? sh.group_rank : sh.group_total - 1 - sh.group_rank;
        const uint32_t blo = sh.blo, bhi = sh.bhi;
        const bool nan_group = sh.nan_group != 0;
        const uint32_t gx = sh.gx_count;
        const uint16_t* rowp = static_cast<const uint16_t*>(a.logits) + static_cast<int64_t>(row) * a.row_stride;
        const bool vec = a.vec_ok != 0;
        auto bin_match = [&](uint32_t bits16) {
            const uint32_t bin = bin_of(bits16);
            return nan_group ? bin_is_nan(bin) : (bin >= blo && bin <= bhi);
        };
        // penalised ids of the group in [lo, hi)
        auto gx_in = [&](uint32_t lo, uint32_t hi) -> uint32_t {
            if (gx == 0) return 0;
            uint32_t a0 = 0, a1 = gx;
            while (a0 < a1) { const uint32_t m = (a0 + a1) >> 1; if (sh.gx_ids[m] < lo) a0 = m + 1; else a1 = m; }
            uint32_t b0 = a0, b1 = gx;
            while (b0 < b1) { const uint32_t m = (b0 + b1) >> 1; if (sh.gx_ids[m] < hi) b0 = m + 1; else b1 = m; }
            return b0 - a0;
        };
        const int nb = (V + 8191) / 8192;
        for (int bi = 0; bi < nb; ++bi) {
            const int batch = fwd ? bi : nb - 1 - bi;
            const int slot = fwd ? tid : kThreads - 1 - tid;  // scan order of this thread's 8 tokens
            const int lo = batch * 8192 + tid * 8;
            uint32_t w4[4] = {0, 0, 0, 0};
            uint32_t valid = 0;  // bit h: token lo + h exists
            if (vec && lo + 8 <= V) {
                const uint4 q = *reinterpret_cast<const uint4*>(rowp + lo);
                w4[0] = q.x; w4[1] = q.y; w4[2] = q.z; w4[3] = q.w;
                valid = 0xFFu;
            } else {
                for (int h = 0; h < 8; ++h) {
                    if (lo + h < V) {
                        w4[h >> 1] |= static_cast<uint32_t>(rowp[lo + h]) << ((h & 1) * 16);
                        valid |= 1u << h;
                    }
                }
            }
            uint32_t mm = 0;  // matching bin tokens
            for (int h = 0; h < 8; ++h) {
                if (((valid >> h) & 1u) && bin_match((w4[h >> 1] >> ((h & 1) * 16)) & 0xFFFFu)) mm |= 1u << h;
            }
            if (mm && pen) {
                const uint32_t word = bitmap[lo >> 5] >> (lo & 31);
                mm &= ~word;
            }
            const uint32_t hi = static_cast<uint32_t>(min(lo + 8, V));
            const uint32_t cnt = static_cast<uint32_t>(__popc(mm)) +
                                 (lo < V ? gx_in(static_cast<uint32_t>(lo), hi) : 0u);
            // exclusive scan in slot order
            const int swave = slot >> 6, slane = slot & 63;
            (void)swave;
            (void)slane;
            // scan by thread index, then mirror for the backward direction
            uint32_t tot;
            const uint32_t ex_fwd = block_excl_scan(cnt, sh.scan, tot);
            const uint32_t ex = fwd ? ex_fwd : tot - ex_fwd - cnt;
            if (want < tot) {
                if (want >= ex && want < ex + cnt) {
                    // this thread holds it: walk its tokens in scan order
                    uint32_t r2 = want - ex;
                    int found = -1;
                    for (int s2 = 0; s2 < 8 && found < 0; ++s2) {
                        const int h = fwd ? s2 : 7 - s2;
                        const uint32_t idx = static_cast<uint32_t>(lo + h);
                        if (!((valid >> h) & 1u)) continue;
                        uint32_t here = (mm >> h) & 1u;
                        if (!here && gx) here = gx_in(idx, idx + 1);
                        if (here) {
                            if (r2 == 0) found = static_cast<int>(idx);
                            else --r2;
                        }
                    }
                    sh.token = found;
                }
                break;
            }
            want -= tot;
        }
    }
    __syncthreads();
    finish(sh.token, aux[item], near ? GE_FLAG_NEAR_BOUNDARY : 0);
}

}  // namespace

hipError_t launch_full_order(const DevArgs& a, hipStream_t stream) {
    if (!a.fo_items) return hipErrorInvalidValue;
    hipLaunchKernelGGL(fo_hist_kernel, dim3(a.rows), dim3(kThreads), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(fo_decide_kernel, dim3(a.rows), dim3(kThreads), 0, stream, a);
    return hipGetLastError();
}

}  // namespace ge
