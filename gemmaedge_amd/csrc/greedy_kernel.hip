// gfx950 greedy kernel of the GemmaEdge token sampler: temperature <= 0,
// the argmax of the final logits (src/generation.cpp:66-70, std::max_element:
// the first maximum, and token 0 when its value is NaN).
//
// One launch covers the batch; each row is split into `cpr` chunks of
// kBlock * EPT logits, one workgroup per chunk. A chunk never evaluates the
// softcap per element: softcap is monotone, so among the tokens that are not
// penalised the largest final value belongs to the largest raw value, and the
// tokens tying with it after the softcap are exactly those whose raw order key
// lies in its tie class [tie_floor(M), M]. Per wave:
//   1. the 16-byte loads of the chunk, and the chunk's bits of the row's
//      history (an LDS bitmap) built while they are in flight;
//   2. M = the wave's largest raw key among unpenalised tokens, its capped
//      value and its tie-class floor (one softcap round on two lanes);
//   3. the lowest index among the wave's unpenalised tokens in the class;
//   4. penalised tokens (those in the history) with their exact final values
//      softcap then penalty, one composite key each.
// The chunk's best composite key (final value descending, index ascending)
// goes to its word of the row's slot area; the last chunk of the row (ticket)
// takes the largest word. Cross-workgroup data is written with agent-scope
// relaxed atomic stores and waited for before the ticket (no L2 writeback).
// On small grids (every workgroup of the launch resident at once, as for one
// row) the chunks instead store words tagged with the row's call epoch and
// leave, and the row's last chunk polls them: one store and one load on the
// last chunk's path instead of a store wait, a ticket and a load.
//
// No MFMA and no LDS staging of logits: a single HBM pass, bound by HBM
// bandwidth for large batches and by the round trips for a single row.
#include <hip/hip_runtime.h>

#include "ge_math.h"
#include "sampler_internal.h"
#include "tie_class.h"
#include "wave_ops.h"

#pragma clang fp contract(off)

namespace ge {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kHistBatch = 8;  // history ids in flight per thread

__device__ __forceinline__ uint64_t max64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// Wave-uniform maximum of a 64-bit key: the largest high word, then the
// largest low word among the lanes holding it.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    const uint32_t hi = wave::max_u32(static_cast<uint32_t>(v >> 32));
    const uint32_t lo = wave::max_u32(static_cast<uint32_t>(v >> 32) == hi ? static_cast<uint32_t>(v) : 0u);
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// d[i] for a run-time i < N (N a power of two): a tree of selects on the
// bits of i, N - 1 selects in all (a private array indexed at run time would
// live in scratch memory).
template <int N>
__device__ __forceinline__ uint32_t pick_word(const uint32_t (&d)[N], uint32_t i) {
    static_assert((N & (N - 1)) == 0, "power of two");
    uint32_t t[N];
#pragma unroll
    for (int j = 0; j < N; ++j) t[j] = d[j];
#pragma unroll
    for (int half = N / 2, b = 0; half >= 1; half /= 2, ++b) {
        const bool hi = ((i >> b) & 1u) != 0u;
#pragma unroll
        for (int j = 0; j < half; ++j) t[j] = hi ? t[2 * j + 1] : t[2 * j];
    }
    return t[0];
}

// Polled chunk words: the composite key's value key, the index in 24 bits
// (vocabularies below 2^24; the largest word is still the best key) and a
// tag: 0x80 | the call epoch's low 7 bits (zero-filled words carry none). A
// chunk with no candidate (key 0) publishes the tag alone.
// The poll is bounded: about 4 s, never reached with every chunk resident
// (they wait for nothing); a wait that runs out gives token -1 with
// GE_FLAG_TIMEOUT. A word stored after that (a chunk stalled for seconds)
// is left in place; its tag makes a later call ignore it until the 7-bit
// epoch wraps (128 calls on the row).
constexpr uint32_t kPollSpins = 1u << 22;
__device__ __forceinline__ uint64_t poll_word(uint64_t b, uint32_t tag) {
    if (b == 0ull) return tag;
    const uint32_t idx = composite_index(b);
    return (static_cast<uint64_t>(composite_key(b)) << 32) | (static_cast<uint64_t>(0xffffffu - idx) << 8) | tag;
}
__device__ __forceinline__ uint64_t poll_composite(uint64_t w) {
    if ((w >> 8) == 0ull) return 0ull;
    return composite(static_cast<uint32_t>(w >> 32), 0xffffffu - static_cast<uint32_t>((w >> 8) & 0xffffffu));
}

__device__ __forceinline__ float load_one(const float* rowp, int i) { return rowp[i]; }
__device__ __forceinline__ float load_one(const uint16_t* rowp, int i) { return bf16_to_f32(rowp[i]); }

template <typename T, int EPT>
__global__ __launch_bounds__(kBlock) void greedy_kernel(DevArgs a) {
    constexpr int W = sizeof(T) == 4 ? 4 : 8;  // elements per 16-byte load
    constexpr int NV = EPT / W;                 // 16-byte loads per thread
    constexpr int NW = EPT * sizeof(T) / 4;     // 32-bit words per thread
    constexpr int CHUNK = kBlock * EPT;
    static_assert(EPT % W == 0 && EPT <= 64, "bad tiling");
    __shared__ uint32_t s_pbits[CHUNK / 32];
    __shared__ uint64_t s_best[kBlock / 64];
    __shared__ uint32_t s_last;

    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int wave = tid >> 6;
    // Block b runs on XCD b % 8; when the rows split evenly over the XCDs,
    // each XCD takes whole rows (as the selection kernel does).
    int bid = static_cast<int>(blockIdx.x);
    if ((a.rows & 7) == 0) bid = (bid & 7) * static_cast<int>(gridDim.x >> 3) + (bid >> 3);
    const int row = bid / a.cpr;
    const int chunk = bid - row * a.cpr;
    if (row_done(a, row)) {
        if (chunk == 0 && tid == 0) skipped_row(a, row);
        return;
    }
    const ge_sample_params p = a.params;  // launched only with shared parameters
    const float cap = p.softcap;
    const float r = p.repetition_penalty;
    const T* rowp = static_cast<const T*>(a.logits) + static_cast<int64_t>(row) * a.row_stride;
    const int V = a.vocab;
    const int c0 = chunk * CHUNK;
    const int cend = min(c0 + CHUNK, V);

    // Slot s of this thread is element c0 + ((s / W) * kBlock + tid) * W + s % W.
    auto elem = [&](int s) { return c0 + ((s / W) * kBlock + tid) * W + (s % W); };

    // 1. The chunk's loads first: they depend on nothing in memory. The
    //    history's length, its first ids, logit 0 (the NaN rule of the last
    //    step) and the row's call epoch (polled words) follow; loads return
    //    in issue order, so the history bitmap below waits for the chunk's
    //    data as well, but no load waits behind another's round trip.
    uint32_t d[NW];
    uint64_t vmask = ~0ull;  // in-range slots
    if (a.vec_ok && c0 + CHUNK <= V) {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const u32x4 q = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(rowp + c0 + (v * kBlock + tid) * W));
            d[4 * v + 0] = q.x;
            d[4 * v + 1] = q.y;
            d[4 * v + 2] = q.z;
            d[4 * v + 3] = q.w;
        }
        if constexpr (EPT < 64) vmask = (1ull << EPT) - 1ull;
    } else {
        vmask = 0ull;
#pragma unroll
        for (int s = 0; s < EPT; ++s) {
            const int e = elem(s);
            if (e < cend) vmask |= 1ull << s;
            const uint32_t bits = e < cend ? f2u(load_one(rowp, e)) : 0u;
            if constexpr (W == 4) {
                d[s] = bits;
            } else if (s % 2 == 0) {
                d[s / 2] = bits >> 16;
            } else {
                d[s / 2] |= bits & 0xffff0000u;
            }
        }
    }
    const int32_t* hist;
    int H;
    row_history(a, row, hist, H);
    const bool pen = H > 0 && !(r == 1.0f);
    int hid[kHistBatch];
    if (pen) {
#pragma unroll
        for (int u = 0; u < kHistBatch; ++u) hid[u] = hist[min(u * kBlock + tid, H - 1)];
    }
    const float x0 = load_one(rowp, 0);
    uint64_t* pw = a.poll ? a.poll + static_cast<int64_t>(row) * kPollStride : nullptr;
    const uint32_t epoch =
        pw ? __hip_atomic_load(reinterpret_cast<const uint32_t*>(&pw[kPollWords]), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT)
           : 0u;
    auto value = [&](int s) -> float {
        if constexpr (W == 4) return u2f(d[s]);
        else return u2f((s % 2 == 0) ? (d[s / 2] << 16) : (d[s / 2] & 0xffff0000u));
    };
    // The chunk's bits of the history (duplicates and ids outside the chunk
    // or the vocabulary are harmless: one bit per token).
    uint64_t pm = 0ull;  // penalised slots of this thread
    if (pen) {
        for (int w = tid; w < CHUNK / 32; w += kBlock) s_pbits[w] = 0u;
        __syncthreads();
        for (int base = 0; base < H; base += kBlock * kHistBatch) {
            if (base > 0) {
#pragma unroll
                for (int u = 0; u < kHistBatch; ++u) hid[u] = hist[min(base + u * kBlock + tid, H - 1)];
            }
#pragma unroll
            for (int u = 0; u < kHistBatch; ++u)
                if (base + u * kBlock + tid < H && hid[u] >= c0 && hid[u] < cend)
                    atomicOr(&s_pbits[(hid[u] - c0) >> 5], 1u << ((hid[u] - c0) & 31));
        }
        __syncthreads();
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int off = (v * kBlock + tid) * W;  // element offset in the chunk
            pm |= static_cast<uint64_t>((s_pbits[off >> 5] >> (off & 31)) & ((1u << W) - 1u)) << (v * W);
        }
    }

    // 2. Unpenalised tokens: the largest raw key M (0 for an empty slot).
    auto key_of = [&](int s) -> uint32_t {
        return (((vmask & ~pm) >> s) & 1ull) ? order_key(value(s)) : 0u;
    };
    uint32_t kmax = 0u;
#pragma unroll
    for (int s = 0; s < EPT; ++s) kmax = max(kmax, key_of(s));
    const uint32_t M = wave::max_u32(kmax);
    // This lane's first penalised slot, if any. A slot index known only at
    // run time selects its word through a tree of selects.
    uint64_t pmv = pm & vmask;
    int sp = -1;
    float xp = 0.0f;
    if (pen && pmv != 0ull) {
        sp = __builtin_ctzll(pmv);
        pmv &= pmv - 1ull;
        const uint32_t w = pick_word(d, static_cast<uint32_t>(W == 4 ? sp : sp / 2));
        xp = W == 4 ? u2f(w) : u2f((sp % 2 == 0) ? (w << 16) : (w & 0xffff0000u));
    }
    // One softcap evaluation per lane: lanes 0 and 1 cap M and the key below
    // it (equal values mean a tie class wider than one key), the others
    // their first penalised value; lanes 0 and 1 cap theirs in a second
    // round, only when one of them has one.
    const bool pair = lane < 2;
    const float sc = softcap(pair ? key_value(M - static_cast<uint32_t>(lane)) : xp, cap);
    float fp = pair ? 0.0f : sc;
    if (pen && __any(pair && sp >= 0)) {
        const float f2 = softcap(xp, cap);
        if (pair) fp = f2;
    }
    uint64_t cand = 0ull;  // this lane's best composite key
    if (M != 0u) {
        const float target = u2f(wave::readlane(f2u(sc), 0));
        const float below = u2f(wave::readlane(f2u(sc), 1));
        const uint32_t L = (cap > 0.0f) ? tie_floor_given(M, cap, target, below) : M;
        // 3. The lowest index among unpenalised tokens in the class [L, M]
        //    (the wave's maximum below picks the lowest).
        uint32_t imin = 0xffffffffu;
#pragma unroll
        for (int s = 0; s < EPT; ++s) {
            const uint32_t k = key_of(s);
            if (k >= L && k != 0u) imin = min(imin, static_cast<uint32_t>(elem(s)));
        }
        if (imin != 0xffffffffu) cand = composite(order_key(cap > 0.0f ? target : key_value(M)), imin);
    }
    // 4. Penalised tokens with their exact final values (softcap, then the
    //    penalty); a lane's further penalised slots, rare, one at a time.
    if (pen && __any(sp >= 0)) {
        if (sp >= 0) cand = max64(cand, composite(order_key(penalize(fp, r)), static_cast<uint32_t>(elem(sp))));
        while (__any(pmv != 0ull)) {
            if (pmv != 0ull) {
                const int s = __builtin_ctzll(pmv);
                pmv &= pmv - 1ull;
                const uint32_t w = pick_word(d, static_cast<uint32_t>(W == 4 ? s : s / 2));
                const float x = W == 4 ? u2f(w) : u2f((s % 2 == 0) ? (w << 16) : (w & 0xffff0000u));
                cand = max64(cand, composite(order_key(penalize(softcap(x, cap), r)), static_cast<uint32_t>(elem(s))));
            }
        }
    }
    const uint64_t best = wave_max_u64(cand);

    // The NaN rule and the outputs (one lane of the row's last chunk):
    // std::max_element (generation.cpp:66-70) keeps index 0 when its final
    // value is NaN (NaN < x is false): its capped value is NaN, or 0 is in
    // the history and the penalty makes it NaN (a NaN penalty, -inf * 0,
    // 0 * inf, inf / inf).
    auto finish = [&](uint64_t b) {
        int32_t token = static_cast<int32_t>(composite_index(b));
        const float f0 = softcap(x0, cap);
        bool nan0 = __builtin_isnan(f0);
        if (!nan0 && pen && __builtin_isnan(penalize(f0, r)))
            for (int j = 0; j < H && !nan0; ++j) nan0 = hist[j] == 0;
        if (nan0) token = 0;
        emit_row(a, row, token, 1.0f, 0);
    };

    if (pw) {
        // Each wave stores its tagged word and leaves (no barrier in the
        // chunk; words [4 c, 4 c + 4) belong to chunk c). The row's last
        // chunk polls every word of the row until all carry this call's tag
        // (each wave stores exactly one, so the wait ends once all have run),
        // clears them and advances the epoch for the next call (the tag guards
        // against a word stored late, after a wait that ran out).
        constexpr int kWpc = kBlock / 64;
        const uint32_t tag = 0x80u | (epoch & 0x7fu);
        if (lane == 0)
            __hip_atomic_store(&pw[chunk * kWpc + wave], poll_word(best, tag), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        if (chunk != a.cpr - 1 || wave != 0) return;
        const int nw = a.cpr * kWpc;  // <= kPollWords
        uint64_t w[kWpc];
        bool all = false;
        for (uint32_t it = 0; it < kPollSpins && !all; ++it) {
            bool mine = true;
#pragma unroll
            for (int j = 0; j < kWpc; ++j) {
                const int q = j * 64 + lane;
                w[j] = q < nw ? __hip_atomic_load(&pw[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                              : static_cast<uint64_t>(tag);
                mine = mine && (static_cast<uint32_t>(w[j]) & 0xffu) == tag;
            }
            all = __ballot(!mine) == 0ull;
            if (!all) __builtin_amdgcn_s_sleep(1);
        }
        // Clear the words (zero carries no tag): a later call whose chunks
        // outnumber this one's never reads a word left from an older call.
        // After a wait that ran out, every word of the row is cleared.
        uint64_t wb = 0ull;
#pragma unroll
        for (int j = 0; j < kWpc; ++j) {
            const int q = j * 64 + lane;
            if (q < nw || !all) __hip_atomic_store(&pw[q], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            wb = max64(wb, w[j]);
        }
        const uint64_t rbest = wave_max_u64(wb);
        if (lane == 0) {
            __hip_atomic_store(&pw[kPollWords], static_cast<uint64_t>(epoch + 1u), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            if (all) finish(poll_composite(rbest));
            else emit_row(a, row, -1, 0.0f, GE_FLAG_TIMEOUT);  // a chunk's word never came: no token
        }
        return;
    }
    if (lane == 0) s_best[wave] = best;
    __syncthreads();

    // Publish the chunk's best, wait for the store, take a ticket; the last
    // chunk of the row reduces the row's words.
    uint64_t* slot = a.slots + static_cast<int64_t>(row) * kSlotWords;
    if (tid == 0) {
        uint64_t b = s_best[0];
#pragma unroll
        for (int w = 1; w < kBlock / 64; ++w) b = max64(b, s_best[w]);
        __hip_atomic_store(&slot[chunk], b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        const uint32_t ticket =
            __hip_atomic_fetch_add(&a.tickets[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = ticket == static_cast<uint32_t>(a.cpr - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (s_last == 0u || wave != 0) return;

    uint64_t b = 0ull;
    for (int c = lane; c < a.cpr; c += 64)
        b = max64(b, __hip_atomic_load(&slot[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    b = wave_max_u64(b);
    if (lane == 0) {
        finish(b);
        a.tickets[row] = 0u;  // ready for the next launch
    }
}

template <typename T, int EPT>
hipError_t launch_t(const DevArgs& a, hipStream_t s) {
    hipLaunchKernelGGL((greedy_kernel<T, EPT>), dim3(static_cast<unsigned>(a.rows * a.cpr)), dim3(kBlock), 0, s, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_greedy(const DevArgs& a, hipStream_t stream, int ept) {
    if (a.dtype == GE_DTYPE_BF16)
        return ept == 16 ? launch_t<uint16_t, 16>(a, stream) : launch_t<uint16_t, 64>(a, stream);
    return ept == 16 ? launch_t<float, 16>(a, stream) : launch_t<float, 64>(a, stream);
}

}  // namespace ge
