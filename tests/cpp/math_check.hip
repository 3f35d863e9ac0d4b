// Test helper: checks the device restatements of glibc's tanhf / expf
// (gemmaedge_amd/csrc/ge_math.h) against the host's libm.
//
//  - ge_test_host_mismatches: the header compiled for the host versus libm,
//    input by input over a range of fp32 bit patterns (multi-threaded);
//  - ge_test_digest: order-independent digests over all 2^32 inputs, in 256
//    blocks of 2^24, computed from libm (impl 0), from the host build of the
//    header (impl 1) or on the GPU from the device build (impl 2). Digest of a
//    block = sum over its inputs x (mod 2^64) of mix(bits(x) << 32 | bits(f(x))),
//    NaN results canonicalised; equal digests over every block mean equal
//    results with overwhelming probability.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdint>
#include <thread>
#include <vector>

#include "../../gemmaedge_amd/csrc/ge_math.h"

namespace {

__host__ __device__ inline uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

__host__ __device__ inline uint32_t canon(float y) {
    const uint32_t b = ge::f2u(y);
    return ((b & 0x7fffffffu) > 0x7f800000u) ? 0x7fc00000u : b;
}

__host__ __device__ inline float eval_ge(int fn, float x) {
    return fn == 0 ? ge::tanhf_fdlibm(x) : ge::expf_glibc(x);
}

inline float eval_libm(int fn, float x) { return fn == 0 ? tanhf(x) : expf(x); }

__global__ void digest_kernel(int fn, uint64_t* out) {
    // 2^32 inputs: block b of the launch covers 2^16 inputs; 256 threads x 256 each.
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) << 16;
    uint64_t acc = 0;
    for (int i = 0; i < 256; ++i) {
        const uint32_t bits = static_cast<uint32_t>(base + static_cast<uint64_t>(i) * 256u + threadIdx.x);
        const float y = eval_ge(fn, ge::u2f(bits));
        acc += mix64((static_cast<uint64_t>(bits) << 32) | canon(y));
    }
    __shared__ uint64_t red[256];
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (threadIdx.x < static_cast<unsigned>(s)) red[threadIdx.x] += red[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) atomicAdd(reinterpret_cast<unsigned long long*>(&out[base >> 24]),
                                    static_cast<unsigned long long>(red[0]));
}

}  // namespace

extern "C" long long ge_test_host_mismatches(int fn, uint32_t lo, uint64_t count, int nthreads) {
    std::atomic<long long> bad{0};
    auto work = [&](int t) {
        long long b = 0;
        for (uint64_t i = static_cast<uint64_t>(t); i < count; i += static_cast<uint64_t>(nthreads)) {
            const float x = ge::u2f(static_cast<uint32_t>(lo + i));
            if (canon(eval_libm(fn, x)) != canon(eval_ge(fn, x))) ++b;
        }
        bad += b;
    };
    std::vector<std::thread> pool;
    for (int t = 0; t < nthreads; ++t) pool.emplace_back(work, t);
    for (auto& th : pool) th.join();
    return bad.load();
}

extern "C" int ge_test_digest(int fn, int impl, uint64_t* out256, int nthreads) {
    for (int b = 0; b < 256; ++b) out256[b] = 0;
    if (impl == 2) {
        uint64_t* d = nullptr;
        if (hipMalloc(&d, 256 * sizeof(uint64_t)) != hipSuccess) return -1;
        if (hipMemset(d, 0, 256 * sizeof(uint64_t)) != hipSuccess) return -1;
        hipLaunchKernelGGL(digest_kernel, dim3(1u << 16), dim3(256), 0, 0, fn, d);
        if (hipGetLastError() != hipSuccess) return -2;
        if (hipMemcpy(out256, d, 256 * sizeof(uint64_t), hipMemcpyDeviceToHost) != hipSuccess) return -3;
        (void)hipFree(d);
        return 0;
    }
    std::vector<uint64_t> part(static_cast<size_t>(nthreads) * 256, 0);
    auto work = [&](int t) {
        for (uint32_t blk = static_cast<uint32_t>(t); blk < 256; blk += static_cast<uint32_t>(nthreads)) {
            uint64_t acc = 0;
            for (uint32_t i = 0; i < (1u << 24); ++i) {
                const uint32_t bits = (blk << 24) | i;
                const float x = ge::u2f(bits);
                const float y = impl == 0 ? eval_libm(fn, x) : eval_ge(fn, x);
                acc += mix64((static_cast<uint64_t>(bits) << 32) | canon(y));
            }
            part[static_cast<size_t>(t) * 256 + blk] = acc;
        }
    };
    std::vector<std::thread> pool;
    for (int t = 0; t < nthreads; ++t) pool.emplace_back(work, t);
    for (auto& th : pool) th.join();
    for (int t = 0; t < nthreads; ++t)
        for (int b = 0; b < 256; ++b) out256[b] += part[static_cast<size_t>(t) * 256 + b];
    return 0;
}

// Number of adjacent non-negative fp32 inputs where libm tanhf decreases
// (0 means monotone on [0, inf]; fdlibm's tanhf is odd, so also on all floats).
extern "C" long long ge_test_tanhf_decreases(int nthreads) {
    std::atomic<long long> bad{0};
    const uint32_t top = 0x7f800000u;  // +inf
    auto work = [&](int t) {
        long long b = 0;
        const uint32_t per = (top + static_cast<uint32_t>(nthreads) - 1) / static_cast<uint32_t>(nthreads);
        const uint32_t lo = per * static_cast<uint32_t>(t);
        const uint32_t hi = lo + per < top ? lo + per : top;
        if (lo >= hi) return;
        float prev = tanhf(ge::u2f(lo));
        for (uint32_t u = lo + 1; u <= hi; ++u) {
            const float y = tanhf(ge::u2f(u));
            if (y < prev) ++b;
            prev = y;
        }
        bad += b;
    };
    std::vector<std::thread> pool;
    for (int t = 0; t < nthreads; ++t) pool.emplace_back(work, t);
    for (auto& th : pool) th.join();
    return bad.load();
}
