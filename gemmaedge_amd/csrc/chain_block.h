// The whole workgroup replays a float or double accumulation over a long list
// of items (runs of equal addends, item i being elements [start(i),
// start(i + 1)) of one addend): the reference's softmax denominator (double),
// top-p cumulative and draw walk (float) over probabilities in sorted order
// (src/generation.cpp:96-97, 105-113, 120-124), for rows whose items number
// up to the vocabulary (f32 logits, where nearly every token is an item of
// its own).
//
// Inside one binade of the accumulator each item is a map of the
// accumulator's parity (chain_math.h ParityMap): ties to even are the only
// steps that depend on the accumulator, and only through its parity. The
// block takes the items in tiles of kThreads * kPer; each thread folds its kPer
// consecutive items into one map, a DPP scan composes the maps across the
// wave, and the waves' totals are composed through LDS. The magnitudes only
// grow along the list, so the first item that would leave the binade, or
// reach the threshold, is found by comparing scanned magnitudes; that item is
// replayed in closed form (chain_math.h asc_run / desc_run) by the thread
// that holds it, and the scan resumes after it in the new binade. A tile thus
// costs one pass per binade crossing in it, and ties cost nothing extra.
//
// Crossings cluster at the head of a list, where the addends are large next to
// the accumulator (a C1-shaped row's double sum crosses at items 2, 5 and 30 of
// its first tile). So a pass first probes: one wave scans the next 64 items the
// same way, and when the first exit lies among them it is replayed at once,
// without the block pass. Probes continue while they find the exits; the
// first that does not hands over to block passes for the rest of the call.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <climits>
#include <cmath>

#include "chain_math.h"
#include "chain_wave.h"
#include "ge_math.h"
#include "wave_ops.h"

#pragma clang fp contract(off)

namespace ge {
namespace bchain {

// Address spaces, for code the compiler may keep out of line: there a plain
// pointer is generic, its accesses become flat instructions, and every wait
// for an LDS access then also waits for every load in flight.
#define GE_GLOBAL __attribute__((address_space(1)))
#define GE_LDS __attribute__((address_space(3)))
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // (HIP's uint4 will not copy from a qualified lvalue)
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kPer = 8;  // consecutive items per thread per tile

// Float accumulator (the top-p cumulative and the draw walk).
struct F32Acc {
    using U = uint32_t;
    static constexpr U kCap = 1u << 28;
    struct Bin {
        U m, lo, hi, tm;
        int uexp;
    };
    __device__ static Bin binade(double s, double thr) {
        const chain::StepBits b = chain::binade_bits(f2u(static_cast<float>(s)));
        return Bin{b.m, b.lo, chain::kHiF, chain::threshold_bits(f2u(static_cast<float>(thr)), b.uexp), b.uexp};
    }
    __device__ static void step(uint32_t ab, int uexp, U& D, bool& tie, bool& odd0, bool& big) {
        chain::step_bits_p(ab, uexp, D, tie, odd0, big);
    }
    __device__ static double rebuild(double s, const Bin&, U m) {
        return static_cast<double>(u2f(chain::rebuild_bits(f2u(static_cast<float>(s)), m)));
    }
    __device__ static uint64_t asc(double& s, double a, uint64_t n, double thr, bool& hit) {
        return chain::asc_run_f32(s, a, n, thr, hit);
    }
    __device__ static uint64_t desc(double& c, double a, uint64_t n, bool& stop) {
        return chain::desc_run_f32(c, a, n, stop);
    }
};

// Double accumulator with float addends (the softmax denominator and the
// near-boundary sums).
struct F64Acc {
    using U = uint64_t;
    static constexpr U kCap = 1ull << 62;
    struct Bin {
        U m, lo, hi, tm;
        int uexp;
    };
    __device__ static Bin binade(double s, double thr) {
        const chain::Binade b = chain::binade_of<double>(s);
        U tm = ~0ull;  // never reached: m + magnitude < 2^63
        if (thr == thr) {
            if (!(thr > 0.0)) tm = 0;
            else if (thr < std::ldexp(1.0, b.uexp + 53)) tm = chain::threshold_m(thr, b.uexp);
        }
        return Bin{b.m, b.lo, b.hi, tm, b.uexp};
    }
    __device__ static void step(uint32_t ab, int uexp, U& D, bool& tie, bool& odd0, bool& big) {
        chain::step_bits64(ab, uexp, D, tie, odd0, big);
    }
    __device__ static double rebuild(double, const Bin& b, U m) {
        return std::ldexp(static_cast<double>(m), b.uexp);
    }
    __device__ static uint64_t asc(double& s, double a, uint64_t n, double thr, bool& hit) {
        return chain::asc_run<double>(s, a, n, thr, hit);
    }
    __device__ static uint64_t desc(double& c, double a, uint64_t n, bool& stop) {
        return chain::desc_run<double>(c, a, n, stop);
    }
};

template <int kWaves>
struct Shared {
    uint64_t me[kWaves];  // per-wave maps (magnitudes from an even / odd start)
    uint64_t mo[kWaves];
    uint64_t pe[kWaves];  // their exclusive composition (the waves before each)
    uint64_t po[kWaves];
    uint64_t te, to;      // and the whole tile's
    int ev[kWaves];       // per-wave first event item, INT_MAX for none
    int last;             // item holding element L - 1, when it lies in the tile
    double rs;            // the event item's replay: accumulator after it,
    uint32_t relem;       // next (or event) element,
    int rhit;             // whether the threshold / stop fired
    double prs[2];        // the same for a probe's event (two buffers: consecutive
    uint32_t prelem[2];   // probes are one barrier apart)
    int prhit[2];
    int pev[2];           // the probe's event item, -1 for none
};

// Items i .. i + kPer - 1: boundaries pb[0..kPer] (clamped to start(G), so
// items past G hold no element) and the bits of their addends, add[i] *
// scale (one float multiplication, so the addend is exactly the float a
// separate scaling pass would have stored; scale 1 leaves it unchanged).
__device__ __forceinline__ void load_tile(const GE_GLOBAL uint32_t* pre, const GE_GLOBAL float* add, float scale, int G,
                                          int i, uint32_t* pb, uint32_t* ab) {
    if (i + kPer <= G) {  // pre has G + 1 entries; i is a multiple of kPer
        const u32x4 p0 = *(const GE_GLOBAL u32x4*)(pre + i);
        const u32x4 p1 = *(const GE_GLOBAL u32x4*)(pre + i + 4);
        pb[0] = p0.x; pb[1] = p0.y; pb[2] = p0.z; pb[3] = p0.w;
        pb[4] = p1.x; pb[5] = p1.y; pb[6] = p1.z; pb[7] = p1.w;
        pb[8] = pre[i + 8];
        const f32x4 a0 = *(const GE_GLOBAL f32x4*)(add + i);
        const f32x4 a1 = *(const GE_GLOBAL f32x4*)(add + i + 4);
        ab[0] = f2u(a0.x * scale); ab[1] = f2u(a0.y * scale); ab[2] = f2u(a0.z * scale); ab[3] = f2u(a0.w * scale);
        ab[4] = f2u(a1.x * scale); ab[5] = f2u(a1.y * scale); ab[6] = f2u(a1.z * scale); ab[7] = f2u(a1.w * scale);
    } else {
#pragma unroll
        for (int j = 0; j <= kPer; ++j) pb[j] = pre[min(i + j, G)];
#pragma unroll
        for (int j = 0; j < kPer; ++j) ab[j] = i + j < G ? f2u(add[i + j] * scale) : 0u;
    }
}

template <bool kDesc, typename Bin, typename U>
__device__ __forceinline__ bool exceeds(const Bin& b, U r) {
    if (kDesc) return b.m < b.lo + r;             // m - r below the binade's exact range
    return b.m + r > b.hi || b.m + r >= b.tm;     // above it, or at the threshold
}

// Replays elements [cp.elem, L) with the whole workgroup (every thread calls
// it with the same arguments; it holds barriers). Semantics as wave_chain_f32
// (chain_wave.h): ascending sums stop at the first element whose sum is >=
// thr (NaN: never), descending ones before the first element with c <= a.
// Returns true on a stop with cp at the stop element; otherwise false with
// cp.elem == L and cp.item holding element L - 1. Requires L <= start(G);
// pre and add 16-byte aligned. Item i's addend is add[i] * scale.
template <typename A, bool kDesc, int kThreads>
__device__ bool block_chain(const uint32_t* pre_p, const float* add_p, float scale, int G, ChainPos& cp_io, uint32_t L,
                            double& s_io, double thr, Shared<kThreads / 64>& sh_p) {
    ChainPos cp = cp_io;  // (locals: the references may be memory of the caller's)
    double s = s_io;
    auto leave = [&](bool r) {
        cp_io = cp;
        s_io = s;
        return r;
    };
    const GE_GLOBAL uint32_t* pre = (const GE_GLOBAL uint32_t*)pre_p;
    const GE_GLOBAL float* add = (const GE_GLOBAL float*)add_p;
    GE_LDS Shared<kThreads / 64>& sh = *(GE_LDS Shared<kThreads / 64>*)&sh_p;
    using U = typename A::U;
    using Map = chain::ParityMap<U>;
    constexpr int kWaves = kThreads / 64;
    constexpr int kTile = kThreads * kPer;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    if (!(cp.elem < L && cp.item < G)) return leave(false);
    int t0 = cp.item / kTile * kTile;
    uint32_t pb[kPer + 1], ab[kPer];
    load_tile(pre, add, scale, G, t0 + tid * kPer, pb, ab);
    bool probe = true;
    int pbuf = 0;
    for (;;) {
        // The next tile's loads are in flight while this one is scanned. They
        // are issued on every tile (the last one loads itself again): with
        // loads issued on one path only, the compiler's wait for this tile's
        // values would cover them too.
        uint32_t npb[kPer + 1], nab[kPer];
        const bool more = t0 + kTile < G;
        load_tile(pre, add, scale, G, (more ? t0 + kTile : t0) + tid * kPer, npb, nab);
        const uint32_t tile_end = pre[min(t0 + kTile, G)];
        const int ibase = t0 + tid * kPer;
        for (;;) {  // one pass per binade the tile's remaining items start in
            const typename A::Bin b = A::binade(s, thr);
            const uint32_t e0 = cp.elem;
            if (probe) {
                // Wave 0 takes items cp.item .. cp.item + 63 of this tile, one
                // per lane, with the pass's maps; the first lane whose item
                // takes the accumulator out of the binade (or to the
                // threshold) is the pass's event, as the block pass would find.
                if (wave == 0) {
                    const int i = cp.item + lane;
                    const int iend = min(t0 + kTile, G);
                    const int ic = min(i, iend - 1);  // clamped: no conditional load
                    const uint32_t lo = max(pre[ic], e0);
                    const uint32_t hi = min(pre[ic + 1], L);
                    const uint32_t abits = f2u(add[ic] * scale);
                    const uint32_t nt = (i < iend && hi > lo) ? hi - lo : 0u;
                    U D;
                    bool tie, odd0, big;
                    A::step(abits, b.uexp, D, tie, odd0, big);
                    const Map f = chain::run_map<U, A::kCap>(nt, D, tie, odd0, big);
                    const Map x = map_wave_excl<U, A::kCap>(f);
                    const U r = chain::apply_from(x, b.m);
                    const U rn = chain::sat_add_cap<U, A::kCap>(r, chain::apply_from(f, static_cast<U>(b.m + r)));
                    const uint64_t em = __ballot(nt != 0u && exceeds<kDesc>(b, rn));
                    if (em == 0ull) {
                        if (lane == 0) sh.pev[pbuf] = -1;
                    } else if (lane == static_cast<int>(__builtin_ctzll(em))) {
                        double sv = A::rebuild(s, b, kDesc ? b.m - r : b.m + r);
                        bool hit = false;
                        const uint64_t used = kDesc ? A::desc(sv, static_cast<double>(u2f(abits)), nt, hit)
                                                    : A::asc(sv, static_cast<double>(u2f(abits)), nt, thr, hit);
                        sh.prs[pbuf] = sv;
                        sh.prhit[pbuf] = hit ? 1 : 0;
                        sh.prelem[pbuf] = hit ? lo + static_cast<uint32_t>(kDesc ? used : used - 1) : hi;
                        sh.pev[pbuf] = i;
                    }
                }
                __syncthreads();
                const int pe = sh.pev[pbuf];
                if (pe >= 0) {
                    s = sh.prs[pbuf];
                    cp.elem = sh.prelem[pbuf];
                    const bool hit = sh.prhit[pbuf] != 0;
                    pbuf ^= 1;
                    if (hit || cp.elem >= L) {
                        cp.item = pe;
                        return leave(hit);
                    }
                    cp.item = pe + 1;
                    continue;
                }
                probe = false;
            }
            Map f{0, 0};
            int last = -1;
#pragma unroll
            for (int j = 0; j < kPer; ++j) {
                const uint32_t lo = max(pb[j], e0);
                const uint32_t hi = min(pb[j + 1], L);
                const uint32_t nt = hi > lo ? hi - lo : 0u;
                U D;
                bool tie, odd0, big;
                A::step(ab[j], b.uexp, D, tie, odd0, big);
                f = chain::compose<U, A::kCap>(f, chain::run_map<U, A::kCap>(nt, D, tie, odd0, big));
                if (nt && hi == L) last = ibase + j;
            }
            const Map x = map_wave_excl<U, A::kCap>(f);
            if (lane == 63) {
                const Map wt = chain::compose<U, A::kCap>(x, f);
                sh.me[wave] = wt.e;
                sh.mo[wave] = wt.o;
            }
            __syncthreads();
            if (wave == 0) {  // one wave composes the waves' maps for all
                const Map t = lane < kWaves ? Map{static_cast<U>(sh.me[lane]), static_cast<U>(sh.mo[lane])} : Map{0, 0};
                const Map ex = map_wave_excl<U, A::kCap>(t);
                if (lane < kWaves) {
                    sh.pe[lane] = ex.e;
                    sh.po[lane] = ex.o;
                }
                if (lane == kWaves - 1) {
                    const Map in = chain::compose<U, A::kCap>(ex, t);
                    sh.te = in.e;
                    sh.to = in.o;
                }
            }
            __syncthreads();
            const Map pw{static_cast<U>(sh.pe[wave]), static_cast<U>(sh.po[wave])};
            const Map tot{static_cast<U>(sh.te), static_cast<U>(sh.to)};
            const U r0 = chain::apply_from(chain::compose<U, A::kCap>(pw, x), b.m);
            const U r_end = chain::sat_add_cap<U, A::kCap>(r0, chain::apply_from(f, static_cast<U>(b.m + r0)));
            int ev = INT_MAX;
            U r_ev = 0;
            if (exceeds<kDesc>(b, r_end)) {  // the first exit may lie in this thread's items
                U r = r0;
#pragma unroll
                for (int j = 0; j < kPer; ++j) {
                    const uint32_t lo = max(pb[j], e0);
                    const uint32_t hi = min(pb[j + 1], L);
                    const uint32_t nt = hi > lo ? hi - lo : 0u;
                    U D;
                    bool tie, odd0, big;
                    A::step(ab[j], b.uexp, D, tie, odd0, big);
                    const Map mj = chain::run_map<U, A::kCap>(nt, D, tie, odd0, big);
                    const U rn = chain::sat_add_cap<U, A::kCap>(r, chain::apply_from(mj, static_cast<U>(b.m + r)));
                    if (ev == INT_MAX && nt && exceeds<kDesc>(b, rn)) {
                        ev = ibase + j;
                        r_ev = r;
                    }
                    r = rn;
                }
            }
            const uint64_t em = __ballot(ev != INT_MAX);
            if (lane == 0) sh.ev[wave] = em ? static_cast<int>(wave::readlane(static_cast<uint32_t>(ev), __builtin_ctzll(em))) : INT_MAX;
            if (last >= 0) sh.last = last;
            __syncthreads();
            int fe = INT_MAX;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) fe = min(fe, sh.ev[w]);
            if (fe == INT_MAX) {
                const U rt = chain::apply_from(tot, b.m);
                s = A::rebuild(s, b, kDesc ? b.m - rt : b.m + rt);
                if (tile_end >= L) {
                    cp.elem = L;
                    cp.item = sh.last;
                    return leave(false);
                }
                cp.elem = tile_end;
                cp.item = t0 + kTile;
                break;
            }
            if (ev == fe) {  // this thread holds the event item: replay it
                const int j = fe - ibase;
                uint32_t lo = 0, hi = 0;
                float a = 0.0f;
#pragma unroll
                for (int q = 0; q < kPer; ++q) {
                    if (q == j) {
                        lo = max(pb[q], e0);
                        hi = min(pb[q + 1], L);
                        a = u2f(ab[q]);
                    }
                }
                const uint32_t nf = hi - lo;
                double sv = A::rebuild(s, b, kDesc ? b.m - r_ev : b.m + r_ev);
                bool hit = false;
                const uint64_t used = kDesc ? A::desc(sv, static_cast<double>(a), nf, hit)
                                            : A::asc(sv, static_cast<double>(a), nf, thr, hit);
                sh.rs = sv;
                sh.rhit = hit ? 1 : 0;
                sh.relem = hit ? lo + static_cast<uint32_t>(kDesc ? used : used - 1) : hi;
            }
            __syncthreads();
            s = sh.rs;
            cp.elem = sh.relem;
            const bool hit = sh.rhit != 0;
            if (hit || cp.elem >= L) {
                cp.item = fe;
                return leave(hit);
            }
            cp.item = fe + 1;
        }
        if (!more) return leave(false);  // unreachable while L <= start(G)
        t0 += kTile;
#pragma unroll
        for (int j = 0; j <= kPer; ++j) pb[j] = npb[j];
#pragma unroll
        for (int j = 0; j < kPer; ++j) ab[j] = nab[j];
    }
}

}  // namespace bchain
}  // namespace ge
