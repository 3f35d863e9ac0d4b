// gfx950 sampling kernels for the GemmaEdge token sampler.
//
// One launch samples `rows` rows. Each row is split into `cpr` chunks of
// kBlock * EPT logits, one workgroup per chunk. A workgroup
//   1. builds its chunk's penalty bitmap in LDS from the row's history,
//   2. streams its chunk from HBM once (16-byte loads, one per thread per
//      vector, consecutive threads on consecutive addresses) into registers and
//      maps each logit to an order key of its RAW value (penalised tokens get
//      key 0 and are handled exactly in step 5),
//   3. takes the maximum of each group of EPT/GPT of its keys and finds, by a
//      two-digit LDS radix histogram, a lower bound tau on the k-th largest of
//      those group maxima; at least k non-penalised logits of the chunk are
//      >= tau, so tau bounds the row's k-th largest raw logit from below,
//   4. lowers tau to the first raw key whose softcapped value equals
//      softcap(tau) (softcap is monotone, so this is exact and keeps every
//      logit that could tie after capping), and appends its logits above that
//      floor to the row's candidate list in global memory,
//   5. increments the row's ticket; the last workgroup of the row merges:
//      tau_row = max over chunks, filters the candidates by its floor,
//      computes exact final values (softcap, then penalty for unique history
//      ids, deduplicated with a per-row bitmap), sorts them by (value desc,
//      index asc) in LDS, and runs the reference's softmax / min-p / top-p /
//      draw with its exact operation order (src/generation.cpp:89-126).
// No MFMA: nothing here is a contraction. The bound is HBM bandwidth.
#include <hip/hip_runtime.h>

#include <climits>

#include "ge_math.h"
#include "sampler_internal.h"

#pragma clang fp contract(off)

namespace ge {
namespace {

__device__ inline uint32_t wave_incl_scan(uint32_t v) {
    const int lane = __lane_id();
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t t = __shfl_up(v, d, 64);
        if (lane >= d) v += t;
    }
    return v;
}

__device__ inline uint32_t wave_max(uint32_t v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v = max(v, (uint32_t)__shfl_xor(v, d, 64));
    return v;
}

__device__ inline int wave_min(int v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v = min(v, __shfl_xor(v, d, 64));
    return v;
}

__device__ inline double wave_sum(double v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
    return v;
}

__device__ inline uint32_t lanes_below(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
}

__device__ inline float load_one(const float* rowp, int i) { return rowp[i]; }
__device__ inline float load_one(const uint16_t* rowp, int i) { return bf16_to_f32(rowp[i]); }

__device__ inline ge_sample_params row_params(const DevArgs& a, int row) {
    return a.row_params ? a.row_params[row] : a.params;
}

__device__ inline void row_history(const DevArgs& a, int row, const int32_t*& h, int& n) {
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
__device__ inline int lsb_exponent(float e) {
    const uint32_t b = f2u(e);
    const uint32_t ex = b >> 23;
    const uint32_t man = b & 0x7fffffu;
    if (ex == 0) return -149 + __builtin_ctz(man);
    return static_cast<int>(ex) - 150 + __builtin_ctz(man | 0x800000u);
}

// Wave 0: hist[256] holds counts per digit; find the digit b (scanning from
// 255 down) where the running count first reaches k. Writes b and the count
// of entries above b.
__device__ inline void find_bin_desc(const uint32_t* hist, uint32_t k, uint32_t* out_bin,
                                     uint32_t* out_above) {
    const int lane = __lane_id();
    const int b0 = 255 - 4 * lane;
    uint32_t h[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) h[i] = hist[b0 - i];
    const uint32_t s = h[0] + h[1] + h[2] + h[3];
    const uint32_t incl = wave_incl_scan(s);
    const uint32_t total = __shfl(incl, 63, 64);
    if (total < k) {  // cannot happen for the callers' k; keep the result defined
        if (lane == 0) {
            *out_bin = 0;
            *out_above = 0;
        }
        return;
    }
    uint32_t c = incl - s;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (c < k && c + h[i] >= k) {
            *out_bin = static_cast<uint32_t>(b0 - i);
            *out_above = c;
        }
        c += h[i];
    }
}

// Lower bound (rounded down to 16 bits) on the k-th largest of the block's
// kBlock*GPT values; 1 <= k <= kBlock*GPT.
template <int GPT>
__device__ uint32_t block_kth_desc16(const uint32_t (&v)[GPT], uint32_t k, uint32_t* s_hist,
                                     uint32_t* s_u32) {
    const int tid = threadIdx.x;
    for (int i = tid; i < 256; i += kBlock) s_hist[i] = 0;
    __syncthreads();
#pragma unroll
    for (int g = 0; g < GPT; ++g) atomicAdd(&s_hist[v[g] >> 24], 1u);
    __syncthreads();
    if (tid < 64) find_bin_desc(s_hist, k, &s_u32[4], &s_u32[5]);
    __syncthreads();
    const uint32_t b1 = s_u32[4];
    const uint32_t k2 = k - s_u32[5];
    for (int i = tid; i < 256; i += kBlock) s_hist[i] = 0;
    __syncthreads();
#pragma unroll
    for (int g = 0; g < GPT; ++g)
        if ((v[g] >> 24) == b1) atomicAdd(&s_hist[(v[g] >> 16) & 255u], 1u);
    __syncthreads();
    if (tid < 64) find_bin_desc(s_hist, k2, &s_u32[4], &s_u32[5]);
    __syncthreads();
    const uint32_t b2 = s_u32[4];
    __syncthreads();
    return (b1 << 24) | (b2 << 16);
}

// Called by one whole wave; every lane returns the same value: the smallest
// raw key x <= tau with softcap(x) == softcap(tau). softcap is monotone
// non-decreasing (glibc tanhf is monotone on all floats), so the keys with
// equal capped value form an interval and a 64-way search finds its floor.
__device__ uint32_t tie_floor(uint32_t tau, float cap) {
    if (!(cap > 0.0f) || tau <= kKeyNegInf) return tau;
    const float target = softcap(key_value(tau), cap);
    const int lane = __lane_id();
    uint32_t hi = tau;  // lowest key known to map to target
    uint32_t lo;        // a key known to map below target
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

// Descending bitonic sort of s[0, n), n a power of two <= kSurvivorCap.
__device__ void bitonic_desc(uint64_t* s, uint32_t n) {
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

struct Shared {
    uint64_t surv[kSurvivorCap];
    float prob[kMaxTopK];
    uint32_t hist[256];
    double f64[kBlock / 64];
    int i32[kBlock / 64];
    uint32_t u32[16];
};

template <typename T>
__device__ void merge_row(const DevArgs& a, Shared& sh, int row, const ge_sample_params& p,
                          bool greedy, uint32_t k, const T* rowp, const int32_t* hist, int H,
                          bool pen, int chunk_len) {
    const int tid = threadIdx.x;
    const int lane = __lane_id();
    const int wave = tid >> 6;
    const int V = a.vocab;
    const float cap = p.softcap;
    const float r = p.repetition_penalty;
    uint32_t* seen = a.seen + static_cast<int64_t>(row) * a.seen_stride;

    // Walks the union of the chunks' candidate lists, one wave per chunk.
    const uint64_t* cand_row = a.cand + static_cast<int64_t>(row) * a.cand_stride;
    auto for_each_candidate = [&](auto&& f) {
        for (int c = wave; c < a.cpr; c += kBlock / 64) {
            const uint32_t n = a.chunk_count[row * kMaxChunks + c];
            const uint64_t* reg = cand_row + static_cast<int64_t>(c) * chunk_len;
            for (uint32_t i = lane; i < n; i += 64) f(reg[i]);
        }
    };

    // Prefilter: the largest chunk bound is a lower bound on the row's k-th
    // largest non-penalised raw logit.
    if (tid == 0) sh.u32[1] = 0;
    __syncthreads();
    if (tid < a.cpr) atomicMax(&sh.u32[1], a.chunk_tau[row * kMaxChunks + tid]);
    __syncthreads();
    if (wave == 0) {
        const uint32_t t = tie_floor(sh.u32[1], cap);
        if (lane == 0) sh.u32[2] = max(t, kKeyNaN);
    }
    __syncthreads();
    const uint32_t thr0 = sh.u32[2];

    // The union holds every logit of the row at or above each chunk's floor,
    // hence the row's top-k raw logits; its k-th largest key is the row's.
    // Two 8-bit radix passes give it rounded down to 16 bits.
    for (int i = tid; i < 256; i += kBlock) sh.hist[i] = 0u;
    __syncthreads();
    for_each_candidate([&](uint64_t e) {
        const uint32_t key = static_cast<uint32_t>(e >> 32);
        if (key >= thr0) atomicAdd(&sh.hist[key >> 24], 1u);
    });
    __syncthreads();
    if (tid < 64) {
        uint32_t s4 = 0;
        for (int i = 0; i < 4; ++i) s4 += sh.hist[tid * 4 + i];
        const uint32_t all = __shfl(wave_incl_scan(s4), 63, 64);
        if (tid == 0) sh.u32[12] = all < k ? 1u : 0u;
        find_bin_desc(sh.hist, k, &sh.u32[4], &sh.u32[5]);
    }
    __syncthreads();
    const bool short_union = sh.u32[12] != 0u;  // fewer than k non-penalised logits
    const uint32_t b1 = sh.u32[4];
    const uint32_t k2 = k - sh.u32[5];
    for (int i = tid; i < 256; i += kBlock) sh.hist[i] = 0u;
    __syncthreads();
    for_each_candidate([&](uint64_t e) {
        const uint32_t key = static_cast<uint32_t>(e >> 32);
        if (key >= thr0 && (key >> 24) == b1) atomicAdd(&sh.hist[(key >> 16) & 255u], 1u);
    });
    __syncthreads();
    if (tid < 64) find_bin_desc(sh.hist, short_union ? 1u : k2, &sh.u32[4], &sh.u32[5]);
    __syncthreads();
    const uint32_t tau_row = short_union ? 0u : ((b1 << 24) | (sh.u32[4] << 16));
    if (wave == 0) {
        const uint32_t t = tie_floor(tau_row, cap);
        if (lane == 0) {
            sh.u32[2] = max(t, thr0);
            sh.u32[3] = 0;
        }
    }
    __syncthreads();
    const uint32_t thr = sh.u32[2];

    // Survivors among the candidates, with exact capped values.
    for_each_candidate([&](uint64_t e) {
        const uint32_t key = static_cast<uint32_t>(e >> 32);
        if (key >= thr) {
            const float f = softcap(key_value(key), cap);
            const uint32_t pos = atomicAdd(&sh.u32[3], 1u);
            if (pos < kSurvivorCap) sh.surv[pos] = composite(order_key(f), static_cast<uint32_t>(e));
        }
    });
    // Penalised tokens: each unique in-range history id once. With r >= 1 the
    // penalty never raises a value, so ids whose raw key is below the floor
    // cannot reach the top-k and are skipped before deduplication.
    const bool prune = r >= 1.0f;
    if (pen) {
        for (int j = tid; j < H; j += kBlock) {
            const int t = hist[j];
            if (t < 0 || t >= V) continue;
            const float raw = load_one(rowp, t);
            if (prune && order_key(raw) < thr) continue;
            const uint32_t bit = 1u << (t & 31);
            const uint32_t old = atomicOr(&seen[t >> 5], bit);
            if (old & bit) continue;
            const float f = penalize(softcap(raw, cap), r);
            const uint32_t pos = atomicAdd(&sh.u32[3], 1u);
            if (pos < kSurvivorCap) sh.surv[pos] = composite(order_key(f), static_cast<uint32_t>(t));
        }
    }
    __syncthreads();
    const uint32_t nsurv = sh.u32[3];
    // Token 0 is penalised (and the penalty is NaN) only if its bit is set.
    const bool zero_seen =
        pen && (__hip_atomic_load(&seen[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 1u);
    __syncthreads();
    if (pen) {
        for (int j = tid; j < H; j += kBlock) {
            const int t = hist[j];
            if (t >= 0 && t < V) seen[t >> 5] = 0u;
        }
    }

    if (nsurv == 0 || nsurv > kSurvivorCap) {
        // More survivors than LDS holds (massive exact ties) or none at all.
        if (tid == 0) {
            a.tokens[row] = -1;
            if (a.probs) a.probs[row] = 0.0f;
            if (a.flags) a.flags[row] = GE_FLAG_UNSUPPORTED;
            a.tickets[row] = 0u;
        }
        return;
    }

    uint32_t n2 = 1;
    while (n2 < nsurv) n2 <<= 1;
    for (uint32_t i = nsurv + tid; i < n2; i += kBlock) sh.surv[i] = 0ull;
    __syncthreads();
    bitonic_desc(sh.surv, n2);
    const uint32_t keff = min(k, nsurv);

    int32_t token = 0;
    float prob = 1.0f;
    int32_t flags = 0;
    if (greedy) {
        // generation.cpp:66-70, std::max_element: first maximum; a NaN at
        // index 0 is never replaced (NaN < x is false), so the answer is 0.
        if (tid == 0) {
            token = static_cast<int32_t>(composite_index(sh.surv[0]));
            bool nan0 = __builtin_isnan(softcap(load_one(rowp, 0), cap));
            if (!nan0 && zero_seen && __builtin_isnan(r)) nan0 = true;
            if (nan0) token = 0;
        }
    } else {
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
        lmin = wave_min(lmin);
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
            // Certified exact: every term is a multiple of 2^m and every
            // partial sum is below 2^(E+2), so 53 bits hold each partial sum
            // exactly when m >= E - 51; then any summation order equals the
            // reference's sequential one. Otherwise replay it sequentially.
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
        if (tid == 0) {
            // generation.cpp:103-115 — min-p / top-p over the sorted probs.
            const float minimum = sh.prob[0] * p.min_p;
            float cumulative = 0.0f;
            uint32_t keep = 0;
            for (; keep < keff; ++keep) {
                const float pk = sh.prob[keep];
                if (pk < minimum && keep > 0) break;
                cumulative += pk;
                if (cumulative >= p.top_p && keep > 0) {
                    ++keep;
                    break;
                }
            }
            keep = max(keep, 1u);
            // generation.cpp:117-126. The reference's `mass` loop adds the same
            // probs in the same order from 0, so it equals `cumulative` bit for bit.
            const float mass = cumulative;
            const float choice0 = a.uniforms[row] * mass + 0.0f;
            float choice = choice0;
            uint32_t pos = keep - 1;
            double c_before = 0.0, c_at = 0.0;
            for (uint32_t i = 0; i < keep; ++i) {
                c_before = c_at;
                c_at += static_cast<double>(sh.prob[i]);
                choice -= sh.prob[i];
                if (choice <= 0.0f) {
                    pos = i;
                    break;
                }
            }
            bool near = false;
            if (pos > 0 && fabs(static_cast<double>(choice0) - c_before) < 1e-6) near = true;
            if (pos + 1 < keep && fabs(static_cast<double>(choice0) - c_at) < 1e-6) near = true;
            token = static_cast<int32_t>(composite_index(sh.surv[pos]));
            prob = sh.prob[pos];
            flags = near ? GE_FLAG_NEAR_BOUNDARY : 0;
        }
    }
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
        a.tickets[row] = 0u;  // ready for the next launch
    }
}

template <typename T, int EPT, int GPT>
__global__ __launch_bounds__(kBlock) void select_kernel(DevArgs a) {
    constexpr int W = sizeof(T) == 4 ? 4 : 8;  // elements per 16-byte load
    constexpr int NV = EPT / W;
    constexpr int CHUNK = kBlock * EPT;
    constexpr int GSZ = EPT / GPT;
    static_assert(EPT % W == 0 && EPT % GPT == 0, "bad tiling");

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

    // 1. Penalty bitmap of this chunk.
    if (pen) {
        for (int w = tid; w < CHUNK / 32; w += kBlock) s_pbits[w] = 0u;
        __syncthreads();
        for (int j = tid; j < H; j += kBlock) {
            const int t = hist[j];
            if (t >= c0 && t < cend) atomicOr(&s_pbits[(t - c0) >> 5], 1u << ((t - c0) & 31));
        }
        __syncthreads();
    }

    // 2. One pass over the chunk: raw order keys in registers.
    uint32_t keys[EPT];
    if (a.vec_ok && c0 + CHUNK <= V) {
        if constexpr (W == 4) {
            float4 q[NV];
#pragma unroll
            for (int v = 0; v < NV; ++v)
                q[v] = *reinterpret_cast<const float4*>(rowp + c0 + (v * kBlock + tid) * 4);
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                keys[v * 4 + 0] = order_key(q[v].x);
                keys[v * 4 + 1] = order_key(q[v].y);
                keys[v * 4 + 2] = order_key(q[v].z);
                keys[v * 4 + 3] = order_key(q[v].w);
            }
        } else {
            uint4 q[NV];
#pragma unroll
            for (int v = 0; v < NV; ++v)
                q[v] = *reinterpret_cast<const uint4*>(rowp + c0 + (v * kBlock + tid) * 8);
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                const uint32_t w4[4] = {q[v].x, q[v].y, q[v].z, q[v].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    keys[v * 8 + 2 * i] = order_key(u2f(w4[i] << 16));
                    keys[v * 8 + 2 * i + 1] = order_key(u2f(w4[i] & 0xffff0000u));
                }
            }
        }
    } else {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
#pragma unroll
            for (int j = 0; j < W; ++j) {
                const int e = c0 + (v * kBlock + tid) * W + j;
                keys[v * W + j] = e < cend ? order_key(load_one(rowp, e)) : kKeyNone;
            }
        }
    }
    if (pen) {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int li = (v * kBlock + tid) * W;  // W divides 32: one bitmap word
            const uint32_t word = s_pbits[li >> 5] >> (li & 31);
#pragma unroll
            for (int j = 0; j < W; ++j)
                if ((word >> j) & 1u) keys[v * W + j] = kKeyNone;
        }
    }

    // 3. Group maxima and the chunk bound tau.
    uint32_t gmax[GPT];
#pragma unroll
    for (int g = 0; g < GPT; ++g) {
        uint32_t m = 0;
#pragma unroll
        for (int j = 0; j < GSZ; ++j) m = max(m, keys[g * GSZ + j]);
        gmax[g] = m;
    }
    uint32_t tau;
    if (k == 1) {
        uint32_t m = 0;
#pragma unroll
        for (int g = 0; g < GPT; ++g) m = max(m, gmax[g]);
        m = wave_max(m);
        if (lane == 0) sh.u32[8 + wave] = m;
        __syncthreads();
        tau = max(max(sh.u32[8], sh.u32[9]), max(sh.u32[10], sh.u32[11]));
    } else {
        tau = block_kth_desc16<GPT>(gmax, k, sh.hist, sh.u32);
    }

    // 4. Tie floor and candidate append.
    if (wave == 0) {
        const uint32_t t = tie_floor(tau, cap);
        if (lane == 0) {
            sh.u32[7] = max(t, kKeyNaN);
            sh.u32[6] = 0u;
        }
    }
    __syncthreads();
    const uint32_t thr = sh.u32[7];
    uint64_t* region = a.cand + static_cast<int64_t>(row) * a.cand_stride + static_cast<int64_t>(c0);
#pragma unroll
    for (int s = 0; s < EPT; ++s) {
        const bool c = keys[s] >= thr;
        const uint64_t m = __ballot(c);
        if (m) {
            uint32_t base = 0;
            if (lane == 0) base = atomicAdd(&sh.u32[6], static_cast<uint32_t>(__popcll(m)));
            base = __shfl(base, 0, 64);
            if (c) {
                const int e = c0 + ((s / W) * kBlock + tid) * W + (s % W);
                region[base + lanes_below(m)] =
                    (static_cast<uint64_t>(keys[s]) << 32) | static_cast<uint32_t>(e);
            }
        }
    }

    // 5. Publish; the last workgroup of the row merges.
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        a.chunk_tau[row * kMaxChunks + chunk] = tau;
        a.chunk_count[row * kMaxChunks + chunk] = sh.u32[6];
        __threadfence();
        const uint32_t ticket = atomicAdd(&a.tickets[row], 1u);
        sh.u32[0] = ticket == static_cast<uint32_t>(a.cpr - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (sh.u32[0] == 0u) return;
    __threadfence();
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
