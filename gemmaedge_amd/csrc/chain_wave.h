// One wave replays a float accumulation over "items" in closed form: item i
// is the run of elements [iv.start(i), iv.start(i + 1)), each adding (or
// subtracting) the same addend iv.addend(i). This is the reference's fp32
// top-p cumulative and the draw's subtract walk (src/generation.cpp:105-113,
// 120-124) over probabilities in sorted order; the full-order kernels use it
// with runs of equal bf16 values, the selection kernel with single elements.
// A View provides start(i), addend(i) and kPerLane (items per lane per step).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "chain_math.h"
#include "ge_math.h"
#include "wave_ops.h"

#pragma clang fp contract(off)

namespace ge {

struct ChainPos {
    int item;       // item holding element `elem`
    uint32_t elem;  // global element index (next to consume, or the event element)
};

template <int kCtrl, int kRowMask, typename U>
__device__ __forceinline__ U dpp_move(U x) {  // lanes without a source read 0
    if constexpr (sizeof(U) == 4) return wave::dpp<kCtrl, kRowMask>(x, 0u);
    else return wave::dpp64<kCtrl, kRowMask>(x, 0ull);
}
template <int kCtrl, int kRowMask, typename U, U kCap>
__device__ __forceinline__ chain::ParityMap<U> map_scan_step(chain::ParityMap<U> v) {
    const chain::ParityMap<U> t{dpp_move<kCtrl, kRowMask>(v.e), dpp_move<kCtrl, kRowMask>(v.o)};
    return chain::compose<U, kCap>(t, v);
}

// Exclusive scan of the lanes' parity maps (chain_math.h ParityMap) in lane
// order, lane 0 getting the identity (0, 0): a wave shift by one lane
// (wave_shr:1), then the row shifts and row broadcasts of wave::incl_u32,
// each composing the map shifted in from lower lanes before the lane's own.
template <typename U, U kCap>
__device__ __forceinline__ chain::ParityMap<U> map_wave_excl(chain::ParityMap<U> f) {
    constexpr int kWaveShr1 = 0x138;
    chain::ParityMap<U> v{dpp_move<kWaveShr1, 0xf>(f.e), dpp_move<kWaveShr1, 0xf>(f.o)};
    v = map_scan_step<wave::kRowShr1, 0xf, U, kCap>(v);
    v = map_scan_step<wave::kRowShr2, 0xf, U, kCap>(v);
    v = map_scan_step<wave::kRowShr4, 0xf, U, kCap>(v);
    v = map_scan_step<wave::kRowShr8, 0xf, U, kCap>(v);
    v = map_scan_step<wave::kRowBcast15, 0xa, U, kCap>(v);
    v = map_scan_step<wave::kRowBcast31, 0xc, U, kCap>(v);
    return v;
}

// Segment totals that let a float chain pass whole steps without replaying
// them (LDS, filled by other waves while the chain runs). Segment s holds the
// items [s * seg, (s + 1) * seg), seg being the chain's items per step. For
// an accumulator in the binade U = 2^uexp, tot[s] is the segment's increment
// in ulps (the sum of each item's elements below the chain's end times its
// rounded addend, capped at 2^24), and bit s of flags marks a segment that
// holds a tie or an addend that leaves the binade (its increment then depends
// on the accumulator). The table is ready once *built reaches need; a table
// with tot == nullptr is none.
struct SkipTable {
    const uint32_t* tot;
    const uint32_t* flags;
    const uint32_t* built;
    uint32_t need;
    int uexp;
};

// The same walk for a float accumulator, in 32-bit integer arithmetic: the
// accumulator is carried as its float bits, each item's increment comes from
// the bit fields of its addend (chain_math.h step_bits), increments are capped
// at 2^24 (more than any binade holds, so the cap never hides an exit) and
// scanned as u32 with DPP. Each lane takes kPerLane consecutive items, so one
// step covers 64 * kPerLane items. With a skip table (ascending chains), steps
// in the table's binade keep to its segments, and a segment that starts at an
// item boundary there, holds no tie and neither leaves the binade, reaches
// the threshold nor holds the chain's end is passed by adding its total.
template <bool kDesc, typename View>
__device__ bool wave_chain_f32(const View& iv, int G, ChainPos& cp, uint32_t L, double& s, double thr,
                               SkipTable skip = SkipTable{nullptr, nullptr, nullptr, 0u, 0}) {
    constexpr int kPerLane = View::kPerLane;
    constexpr int kSeg = 64 * kPerLane;
    constexpr uint32_t kCap = 0x1000000u;
    const int lane = __lane_id();
    const uint32_t tb = f2u(static_cast<float>(thr));
    uint32_t sb = f2u(static_cast<float>(s));
    bool ready = false;  // the table was seen complete (it stays so)
    while (cp.elem < L && cp.item < G) {
        const chain::StepBits bb = chain::binade_bits(sb);
        // in the table's binade: steps keep to its segments, and a segment
        // may be passed whole
        const bool in_table = skip.tot != nullptr && bb.uexp == skip.uexp;
        if (in_table && cp.item % kSeg == 0 && !ready)
            ready = __hip_atomic_load(skip.built, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= skip.need;
        if (in_table && cp.item % kSeg == 0 && ready) {
            const int sg = cp.item / kSeg;
            const int next = min(cp.item + kSeg, G);
            if (!((skip.flags[sg >> 5] >> (sg & 31)) & 1u) && cp.elem == iv.start(cp.item)) {
                const uint32_t m2 = bb.m + skip.tot[sg];  // <= 2^24 + 2^24
                const uint32_t tile_end = iv.start(next);
                if (m2 <= chain::kHiF && m2 < chain::threshold_bits(tb, bb.uexp) && tile_end < L) {
                    sb = (sb >> 23) <= 1u ? m2 : ((sb & 0x7F800000u) | (m2 & 0x7FFFFFu));
                    cp.item = next;
                    cp.elem = tile_end;
                    continue;
                }
            }
        }
        // the step's items: [cp.item, iend), within one segment when skipping
        const int iend = in_table ? min(G, (cp.item / kSeg + 1) * kSeg) : min(G, cp.item + kSeg);
        const int i0 = cp.item + lane * kPerLane;
        uint32_t bound[kPerLane + 1];
#pragma unroll
        for (int j = 0; j <= kPerLane; ++j) bound[j] = iv.start(min(i0 + j, iend));
        uint32_t ab[kPerLane];
#pragma unroll
        for (int j = 0; j < kPerLane; ++j) {  // G >= 1: the clamped read is in range
            const uint32_t v = f2u(iv.addend(min(i0 + j, G - 1)));
            ab[j] = i0 + j < iend ? v : 0u;
        }
        const uint32_t tm = kDesc ? 0u : chain::threshold_bits(tb, bb.uexp);
        uint32_t nt[kPerLane], lo_e[kPerLane], pre_in[kPerLane + 1];
        bool evj[kPerLane];
        pre_in[0] = 0;
#pragma unroll
        for (int j = 0; j < kPerLane; ++j) {
            lo_e[j] = max(bound[j], cp.elem);
            const uint32_t hi_e = min(bound[j + 1], L);
            nt[j] = hi_e > lo_e[j] ? hi_e - lo_e[j] : 0u;
            uint32_t D;
            bool tie, big;
            chain::step_bits(ab[j], bb.uexp, D, tie, big);
            const uint32_t lo32 = nt[j] * D;
            const uint32_t capped = (__umulhi(nt[j], D) != 0u || lo32 > kCap) ? kCap : lo32;
            const uint32_t tot = big ? 0u : capped;  // nt = 0 gives 0
            pre_in[j + 1] = pre_in[j] + tot;  // <= 4 * 2^24
            evj[j] = nt[j] && (big || tie);
        }
        const uint32_t lane_tot = min(pre_in[kPerLane], kCap);
        const uint32_t excl = wave::incl_add(lane_tot) - lane_tot;  // <= 2^30
        int jf = kPerLane;
#pragma unroll
        for (int j = kPerLane - 1; j >= 0; --j) {
            const uint32_t after = excl + pre_in[j + 1];
            bool e = evj[j];
            if (nt[j]) e = e || (kDesc ? bb.m < bb.lo + after : (bb.m + after > chain::kHiF || bb.m + after >= tm));
            if (e) jf = j;
        }
        const uint64_t evmask = __ballot(jf < kPerLane);
        const int f = evmask ? static_cast<int>(__builtin_ctzll(evmask)) : 64;
        if (f == 64) {
            const uint32_t total = wave::readlane(excl + lane_tot, 63);
            const uint32_t m2 = kDesc ? bb.m - total : bb.m + total;
            sb = (sb >> 23) <= 1u ? m2 : ((sb & 0x7F800000u) | (m2 & 0x7FFFFFu));
            const int next = iend;
            const uint32_t tile_end = iv.start(next);
            if (tile_end >= L) {  // the last element lies in this step
                int where = -1;
#pragma unroll
                for (int j = 0; j < kPerLane; ++j)
                    if (nt[j] && lo_e[j] + nt[j] == L) where = i0 + j;
                const uint64_t lm = __ballot(where >= 0);
                cp.item = static_cast<int>(wave::readlane(static_cast<uint32_t>(where), static_cast<int>(__builtin_ctzll(lm))));
                cp.elem = L;
                s = static_cast<double>(u2f(sb));
                return false;
            }
            cp.elem = tile_end;
            cp.item = next;
            continue;
        }
        // lanes before f, and items of lane f before its event item, in one step
        const int jfu = static_cast<int>(wave::readlane(static_cast<uint32_t>(jf), f));
        uint32_t before_in = 0, lo_f = 0, n_f = 0, a_f = 0;
#pragma unroll
        for (int j = 0; j < kPerLane; ++j) {
            if (j == jfu) {
                before_in = pre_in[j];
                lo_f = lo_e[j];
                n_f = nt[j];
                a_f = ab[j];
            }
        }
        const uint32_t before = wave::readlane(excl + before_in, f);
        const uint32_t m2 = kDesc ? bb.m - before : bb.m + before;
        sb = (sb >> 23) <= 1u ? m2 : ((sb & 0x7F800000u) | (m2 & 0x7FFFFFu));
        cp.item = cp.item + f * kPerLane + jfu;
        cp.elem = wave::readlane(lo_f, f);
        const uint32_t nf = wave::readlane(n_f, f);
        const double af = static_cast<double>(u2f(wave::readlane(a_f, f)));
        double sd = static_cast<double>(u2f(sb));
        bool evt = false;
        const uint64_t used = kDesc ? chain::desc_run_f32(sd, af, nf, evt)
                                    : chain::asc_run_f32(sd, af, nf, thr, evt);
        sb = f2u(static_cast<float>(sd));
        if (evt) {
            cp.elem += static_cast<uint32_t>(kDesc ? used : used - 1);
            s = sd;
            return true;
        }
        cp.elem += nf;
        if (cp.elem >= L) {
            s = sd;
            return false;
        }
        cp.item += 1;
    }
    s = static_cast<double>(u2f(sb));
    return false;
}

}  // namespace ge
