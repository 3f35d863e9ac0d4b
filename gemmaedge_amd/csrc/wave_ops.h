// Wave64 building blocks for gfx950 that stay in the VALU / SALU: DPP row
// shifts and row broadcasts for scans and reductions, v_readlane for
// broadcasts, ballots for counting. __shfl and friends lower to ds_bpermute,
// a round trip through the LDS crossbar (on the order of 100 cycles), and a
// chain of them (a 6-step butterfly, a 21-stage sort) is a latency chain; the
// forms here cost a few cycles per step.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ge {
namespace wave {

// DPP controls (GCN / CDNA encoding).
constexpr int kRowShr1 = 0x111, kRowShr2 = 0x112, kRowShr4 = 0x114, kRowShr8 = 0x118;
constexpr int kRowBcast15 = 0x142, kRowBcast31 = 0x143;

// x moved by the DPP pattern; lanes with no source (or in a row the row mask
// leaves out) read `fill`.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint32_t dpp(uint32_t x, uint32_t fill) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(static_cast<int>(fill), static_cast<int>(x), kCtrl, kRowMask, 0xf, false));
}

__device__ __forceinline__ uint32_t readlane(uint32_t v, int lane) {
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), lane));
}
__device__ __forceinline__ uint64_t readlane64(uint64_t v, int lane) {
    return (static_cast<uint64_t>(readlane(static_cast<uint32_t>(v >> 32), lane)) << 32) |
           readlane(static_cast<uint32_t>(v), lane);
}
__device__ __forceinline__ double readlane_f64(double v, int lane) {
    return __builtin_bit_cast(double, readlane64(__builtin_bit_cast(uint64_t, v), lane));
}

// Inclusive scan pattern: rows of 16 by shifts 1, 2, 4, 8, then row totals
// carried into rows 1 and 3 (row_bcast 15) and into rows 2 and 3 (row_bcast
// 31). `op` must be associative with `id` its identity; lane 63 ends with the
// whole wave's result.
template <typename Op>
__device__ __forceinline__ uint32_t incl_u32(uint32_t v, uint32_t id, Op op) {
    v = op(v, dpp<kRowShr1, 0xf>(v, id));
    v = op(v, dpp<kRowShr2, 0xf>(v, id));
    v = op(v, dpp<kRowShr4, 0xf>(v, id));
    v = op(v, dpp<kRowShr8, 0xf>(v, id));
    v = op(v, dpp<kRowBcast15, 0xa>(v, id));
    v = op(v, dpp<kRowBcast31, 0xc>(v, id));
    return v;
}

__device__ __forceinline__ uint32_t incl_add(uint32_t v) {
    return incl_u32(v, 0u, [](uint32_t a, uint32_t b) { return a + b; });
}
// Wave-uniform reductions.
__device__ __forceinline__ uint32_t max_u32(uint32_t v) {
    return readlane(incl_u32(v, 0u, [](uint32_t a, uint32_t b) { return a > b ? a : b; }), 63);
}
__device__ __forceinline__ uint32_t min_u32(uint32_t v) {
    return readlane(incl_u32(v, 0xffffffffu, [](uint32_t a, uint32_t b) { return a < b ? a : b; }), 63);
}
__device__ __forceinline__ int min_i32(int v) {
    // Signed order through the sign-flipped unsigned order.
    const uint32_t u = static_cast<uint32_t>(v) ^ 0x80000000u;
    return static_cast<int>(min_u32(u) ^ 0x80000000u);
}

template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint64_t dpp64(uint64_t x, uint64_t fill) {
    const uint32_t lo = dpp<kCtrl, kRowMask>(static_cast<uint32_t>(x), static_cast<uint32_t>(fill));
    const uint32_t hi = dpp<kCtrl, kRowMask>(static_cast<uint32_t>(x >> 32), static_cast<uint32_t>(fill >> 32));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}
// Sum in the scan's order (not the reference's): callers use it only where
// every order gives the same result, or as a certificate check.
__device__ __forceinline__ double sum_f64(double v) {
    auto d = [](double x, auto ctl) -> double {
        return __builtin_bit_cast(double, ctl(__builtin_bit_cast(uint64_t, x)));
    };
    v += d(v, [](uint64_t x) { return dpp64<kRowShr1, 0xf>(x, 0); });
    v += d(v, [](uint64_t x) { return dpp64<kRowShr2, 0xf>(x, 0); });
    v += d(v, [](uint64_t x) { return dpp64<kRowShr4, 0xf>(x, 0); });
    v += d(v, [](uint64_t x) { return dpp64<kRowShr8, 0xf>(x, 0); });
    v += d(v, [](uint64_t x) { return dpp64<kRowBcast15, 0xa>(x, 0); });
    v += d(v, [](uint64_t x) { return dpp64<kRowBcast31, 0xc>(x, 0); });
    return readlane_f64(v, 63);
}

// Inclusive prefix sum (lane i: v_0 + ... + v_i) in the scan's association
// order; callers use it only where every order gives the same sums.
__device__ __forceinline__ double incl_f64(double v) {
    auto sh = [](double x, auto ctl) -> double {
        return __builtin_bit_cast(double, ctl(__builtin_bit_cast(uint64_t, x)));
    };
    v += sh(v, [](uint64_t x) { return dpp64<kRowShr1, 0xf>(x, 0); });
    v += sh(v, [](uint64_t x) { return dpp64<kRowShr2, 0xf>(x, 0); });
    v += sh(v, [](uint64_t x) { return dpp64<kRowShr4, 0xf>(x, 0); });
    v += sh(v, [](uint64_t x) { return dpp64<kRowShr8, 0xf>(x, 0); });
    v += sh(v, [](uint64_t x) { return dpp64<kRowBcast15, 0xa>(x, 0); });
    v += sh(v, [](uint64_t x) { return dpp64<kRowBcast31, 0xc>(x, 0); });
    return v;
}

// The t-th largest (1 <= t <= 64) of the 64 lanes' keys, wave-uniform:
// the largest x with at least t lanes holding a key >= x, found bit by bit
// with ballots (one compare per bit; the count is a scalar popcount).
__device__ __forceinline__ uint32_t kth_largest(uint32_t key, uint32_t t) {
    uint32_t x = 0u;
#pragma unroll
    for (int b = 31; b >= 0; --b) {
        const uint32_t c = x | (1u << b);
        if (static_cast<uint32_t>(__popcll(__ballot(key >= c))) >= t) x = c;
    }
    return x;
}

}  // namespace wave
}  // namespace ge
