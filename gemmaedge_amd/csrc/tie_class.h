// Softcap tie classes of raw logits (gfx950 device code, one whole wave).
//
// softcap(l) = c * tanhf(l / c) (src/generation.cpp:431-437) is monotone
// non-decreasing (glibc tanhf is monotone on every float), so the raw order
// keys whose capped values are equal form an interval. The selection and
// greedy kernels order by raw keys and need the ends of the interval that
// holds a given key: every key in it ties after the softcap, and the lowest
// token index among them comes first.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ge_math.h"
#include "wave_ops.h"

namespace ge {

// Called by one whole wave; every lane returns the same value: the smallest
// raw key x <= tau with softcap(x) == softcap(tau). softcap is monotone
// non-decreasing (glibc tanhf is monotone on all floats), so the keys with
// equal capped value form an interval. Usually tau-1 already caps lower and
// one evaluation round decides; otherwise a 64-way search finds the floor.
// tie_floor with its first evaluation supplied: target = softcap(tau),
// below = softcap(tau - 1) (both wave-uniform).
__device__ __forceinline__ uint32_t tie_floor_given(uint32_t tau, float cap, float target, float below) {
    if (!(cap > 0.0f) || tau <= kKeyNegInf) return tau;
    if (below != target) return tau;
    const int lane = __lane_id();
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
            const uint32_t xj = wave::readlane(x, j);
            const uint32_t xp = wave::readlane(x, j > 0 ? j - 1 : 0);
            lo = xj;
            hi = j > 0 ? xp : hi;
            break;
        }
        hi = wave::readlane(x, 63);
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
        const uint32_t xj = wave::readlane(x, j);
        const uint32_t xp = wave::readlane(x, j > 0 ? j - 1 : 0);
        lo = j > 0 ? xp : lo;
        hi = xj;
    }
    return hi;
}

__device__ __forceinline__ uint32_t tie_floor(uint32_t tau, float cap) {
    if (!(cap > 0.0f) || tau <= kKeyNegInf) return tau;
    const int lane = __lane_id();
    const float s01 = softcap(key_value(tau - static_cast<uint32_t>(lane & 1)), cap);
    return tie_floor_given(tau, cap, u2f(wave::readlane(f2u(s01), 0)), u2f(wave::readlane(f2u(s01), 1)));
}

// Mirror of tie_floor: the largest raw key x >= r with softcap(x) ==
// softcap(r). One whole wave; every lane returns the same value.
__device__ __forceinline__ uint32_t tie_ceil(uint32_t r, float cap) {
    if (!(cap > 0.0f) || r < kKeyNegInf || r >= kKeyPosInf) return r;
    const int lane = __lane_id();
    const float s01 = softcap(key_value(r + static_cast<uint32_t>(lane & 1)), cap);
    const float target = u2f(wave::readlane(f2u(s01), 0));
    if (u2f(wave::readlane(f2u(s01), 1)) != target) return r;
    uint32_t lo = r + 1;  // highest key known to map to target
    uint32_t hi;          // a key known to map above target
    uint64_t step = 1;
    for (;;) {
        const uint64_t off = static_cast<uint64_t>(lane + 1) * step;
        const uint32_t x = (static_cast<uint64_t>(kKeyPosInf - lo) > off)
                               ? lo + static_cast<uint32_t>(off)
                               : kKeyPosInf;
        const bool eq = softcap(key_value(x), cap) == target;
        const uint64_t ne = __ballot(!eq);
        if (ne) {
            const int j = __ffsll(static_cast<unsigned long long>(ne)) - 1;
            const uint32_t xj = wave::readlane(x, j);
            const uint32_t xp = wave::readlane(x, j > 0 ? j - 1 : 0);
            hi = xj;
            lo = j > 0 ? xp : lo;
            break;
        }
        lo = wave::readlane(x, 63);
        if (lo == kKeyPosInf) return kKeyPosInf;
        step *= 64;
    }
    while (hi - lo > 1) {
        const uint32_t span = hi - lo;
        const uint32_t s = (span + 63u) / 64u;
        const uint64_t off = static_cast<uint64_t>(lane + 1) * s;
        const uint32_t x = off < span ? lo + static_cast<uint32_t>(off) : hi;
        const bool eq = softcap(key_value(x), cap) == target;
        const uint64_t nm = __ballot(!eq);  // non-empty: lanes probing hi differ
        const int j = __ffsll(static_cast<unsigned long long>(nm)) - 1;
        const uint32_t xj = wave::readlane(x, j);
        const uint32_t xp = wave::readlane(x, j > 0 ? j - 1 : 0);
        lo = j > 0 ? xp : lo;
        hi = xj;
    }
    return lo;
}

}  // namespace ge
