// Exact replay of a sequential floating-point accumulation in closed form.
//
// The reference's softmax denominator (double), its top-p cumulative and the
// subtract walk of its draw (float) are left-to-right sums over the
// probabilities in sorted order (src/generation.cpp:96-97, 105-113, 120-124).
// When many consecutive terms are equal — every token of one bf16 value has
// the same probability — the same addend a is applied n times. Inside one
// binade of the accumulator (all values sharing one ulp U) each step changes
// the accumulator by the same whole number of ulps, D = round(a / U), so n
// steps collapse to one multiplication:
//
//   ascending   s + a  ->  s + D*U   valid while the exact result stays below
//                                    the binade's top (m + D <= 2^P - 1);
//   descending  c - a  ->  c - D*U   valid while it stays above the binade's
//                                    bottom (m - D >= 2^(P-1) + 1).
//
// (m = s / U is an integer and P is the precision: 24 for float, 53 for
// double.) Ties to even make a step depend on the parity of m when a / U has
// fraction exactly 1/2: the result is the even one of the two neighbours, so
// from an even m every step adds (or removes) the even one of floor(a/U) and
// floor(a/U) + 1, and from an odd m one ordinary rounded operation makes m
// even first. The step
// that leaves the binade is also taken as an ordinary operation, after which
// the next binade's ulp applies. A run of n equal addends therefore costs
// O(binades crossed + ties) operations instead of O(n).
//
// Everything is held exactly in double: accumulator values are float or
// double numbers, m < 2^53, and a / U is a power-of-two scaling of a float.
// Host and device share this code; tests/cpp/chain_check.hip compares it with
// plain loops on the CPU.
#pragma once

#include <stdint.h>

#include <cmath>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define GE_CHAIN_HD __host__ __device__ inline
#else
#define GE_CHAIN_HD inline
#endif

#pragma clang fp contract(off)

namespace ge {
namespace chain {

template <typename Acc>
struct AccTraits;
template <>
struct AccTraits<float> {
    static constexpr int P = 24;          // significand bits
    static constexpr int kMinNormalExp = -126;
};
template <>
struct AccTraits<double> {
    static constexpr int P = 53;
    static constexpr int kMinNormalExp = -1022;
};

constexpr uint64_t kNone = ~static_cast<uint64_t>(0);

struct Binade {
    int uexp;     // ulp U = 2^uexp
    uint64_t m;   // accumulator / U
    uint64_t hi;  // largest m an ascending step may produce and stay exact
    uint64_t lo;  // smallest m a descending step may produce and stay exact
};

GE_CHAIN_HD uint64_t dbits(double d) { return __builtin_bit_cast(uint64_t, d); }

// Binade of s >= 0 (finite, representable in Acc). Values below the first
// normal binade share its ulp, so [0, 2^(kMinNormalExp+1)) is one region in
// which every operation on Acc numbers is exact.
template <typename Acc>
GE_CHAIN_HD Binade binade_of(double s) {
    constexpr int P = AccTraits<Acc>::P;
    Binade b;
    b.hi = (static_cast<uint64_t>(1) << P) - 1;
    const int ex = static_cast<int>((dbits(s) >> 52) & 0x7ff);
    const int e = ex - 1023;  // s in [2^e, 2^(e+1)) for normal doubles
    if (s == 0.0 || ex == 0 || e <= AccTraits<Acc>::kMinNormalExp) {
        b.uexp = AccTraits<Acc>::kMinNormalExp - (P - 1);
        b.lo = 1;
    } else {
        b.uexp = e - (P - 1);
        b.lo = (static_cast<uint64_t>(1) << (P - 1)) + 1;
    }
    b.m = static_cast<uint64_t>(std::ldexp(s, -b.uexp));
    return b;
}

// Increment of one step of addend a >= 0 in binade b: D = a / U rounded to
// the nearest integer. tie: the fraction is exactly 1/2, and D is then the
// even neighbour (the increment from an even m); big: a alone reaches the
// binade's top (the step leaves the binade at once).
struct Step {
    uint64_t D;
    bool tie;
    bool big;
};

template <typename Acc>
GE_CHAIN_HD Step step_of(const Binade& b, double a) {
    constexpr int P = AccTraits<Acc>::P;
    Step st{0, false, false};
    if (a >= std::ldexp(1.0, b.uexp + P)) {
        st.big = true;
        return st;
    }
    const double A = std::ldexp(a, -b.uexp);
    const double D0 = std::floor(A);
    const double f = A - D0;
    const uint64_t d0 = static_cast<uint64_t>(D0);
    st.tie = f == 0.5;
    st.D = st.tie ? d0 + (d0 & 1u) : d0 + (f > 0.5 ? 1u : 0u);
    return st;
}

template <typename Acc>
GE_CHAIN_HD double add_once(double s, double a) {
    return static_cast<double>(static_cast<Acc>(s) + static_cast<Acc>(a));
}
template <typename Acc>
GE_CHAIN_HD double sub_once(double s, double a) {
    return static_cast<double>(static_cast<Acc>(s) - static_cast<Acc>(a));
}

// floor(a / b) for a < 2^54, 1 <= b: a double quotient corrected to the exact
// one (64-bit integer division is a long software sequence on the GPU).
GE_CHAIN_HD uint64_t udiv(uint64_t a, uint64_t b) {
    uint64_t q = static_cast<uint64_t>(static_cast<double>(a) / static_cast<double>(b));
    while (q * b > a) --q;
    while ((q + 1) * b <= a) ++q;
    return q;
}

// Smallest m whose value m * 2^uexp is >= thr (thr > 0, below the binade top).
GE_CHAIN_HD uint64_t threshold_m(double thr, int uexp) {
    return static_cast<uint64_t>(std::ceil(std::ldexp(thr, -uexp)));
}

// s <- s + a applied n times in Acc arithmetic, as a left-to-right loop would.
// thr: stop at the first step whose result is >= thr (NaN: never). Returns the
// number of steps taken (including the stopping one); hit tells whether the
// threshold stopped it.
template <typename Acc>
GE_CHAIN_HD uint64_t asc_run(double& s, double a, uint64_t n, double thr, bool& hit) {
    constexpr int P = AccTraits<Acc>::P;
    hit = false;
    uint64_t done = 0;
    while (done < n) {
        if (!(a > 0.0)) {  // a == 0: the value never changes
            if (s >= thr) {
                hit = true;
                return done + 1;
            }
            return n;
        }
        if (s == 0.0) {    // 0 + a == a exactly
            s = add_once<Acc>(s, a);
            ++done;
            if (s >= thr) {
                hit = true;
                return done;
            }
            continue;
        }
        Binade b = binade_of<Acc>(s);
        const Step st = step_of<Acc>(b, a);
        if (st.big || (st.tie && (b.m & 1u))) {
            s = add_once<Acc>(s, a);
            ++done;
            if (s >= thr) {
                hit = true;
                return done;
            }
            continue;
        }
        const uint64_t rem = n - done;
        const uint64_t jv = st.D ? udiv(b.hi - b.m, st.D) : kNone;  // steps that stay exact
        uint64_t jh = kNone;                                     // steps to reach thr
        if (thr == thr) {
            if (!(thr > 0.0)) {
                jh = 1;
            } else if (thr < std::ldexp(1.0, b.uexp + P)) {
                const uint64_t tm = threshold_m(thr, b.uexp);
                if (b.m >= tm) jh = 1;
                else if (st.D) jh = udiv(tm - b.m + st.D - 1, st.D);
            }
        }
        uint64_t j = rem < jv ? rem : jv;
        if (jh < j) j = jh;
        b.m += j * st.D;
        s = std::ldexp(static_cast<double>(b.m), b.uexp);
        done += j;
        if (j == jh) {
            hit = true;
            return done;
        }
        if (done < n) {    // the step that leaves the binade
            s = add_once<Acc>(s, a);
            ++done;
            if (s >= thr) {
                hit = true;
                return done;
            }
        }
    }
    return n;
}

// c <- c - a applied up to n times in Acc arithmetic, stopping before the
// first step at which c <= a (the reference's `choice -= p; if (choice <= 0)`:
// c - a rounds to <= 0 exactly when c <= a). Returns the number of steps
// taken before the stop (stop = true), or n.
template <typename Acc>
GE_CHAIN_HD uint64_t desc_run(double& c, double a, uint64_t n, bool& stop) {
    stop = false;
    uint64_t done = 0;
    while (done < n) {
        if (c <= a) {
            stop = true;
            return done;
        }
        if (!(a > 0.0)) return n;  // c - 0 == c
        Binade b = binade_of<Acc>(c);
        const Step st = step_of<Acc>(b, a);  // a < c, so never big
        if (st.tie && (b.m & 1u)) {
            c = sub_once<Acc>(c, a);
            ++done;
            continue;
        }
        if (st.D == 0 && b.m >= b.lo) return n;  // rounds back to c forever
        const uint64_t jv = (st.D && b.m >= b.lo) ? udiv(b.m - b.lo, st.D) : 0;
        const uint64_t rem = n - done;
        const uint64_t j = rem < jv ? rem : jv;
        b.m -= j * st.D;
        c = std::ldexp(static_cast<double>(b.m), b.uexp);
        done += j;
        if (done < n) {    // the step that leaves the binade, or a stop
            if (c <= a) {
                stop = true;
                return done;
            }
            c = sub_once<Acc>(c, a);
            ++done;
        }
    }
    return n;
}

// ---- float accumulator: one step from the bit fields ------------------------
//
// For a float accumulator with bits sb (value >= 0) and a float addend with
// bits ab (>= 0), the binade, a / U rounded, the tie flag and the
// threshold in ulps follow from the exponent and significand fields with
// shifts alone (no floating-point arithmetic).

struct StepBits {
    uint32_t m;     // accumulator / U
    uint32_t lo;    // smallest m a descending step may produce and stay exact
    int uexp;       // U = 2^uexp
};

GE_CHAIN_HD StepBits binade_bits(uint32_t sb) {
    const uint32_t ex = sb >> 23;
    StepBits b;
    if (ex <= 1u) {  // subnormals and the first normal binade: U = 2^-149
        b.m = sb & 0x00FFFFFFu;
        b.lo = 1u;
        b.uexp = -149;
    } else {
        b.m = (sb & 0x7FFFFFu) | 0x800000u;
        b.lo = 0x800001u;
        b.uexp = static_cast<int>(ex) - 150;
    }
    return b;
}

// Significand and exponent of a non-negative float: value = man * 2^(e - 150).
GE_CHAIN_HD void float_fields(uint32_t bits, uint32_t& man, int& e) {
    const uint32_t ex = bits >> 23;
    man = ex ? ((bits & 0x7FFFFFu) | 0x800000u) : (bits & 0x7FFFFFu);
    e = ex ? static_cast<int>(ex) : 1;
}

// D = round(a / U) with the tie flag (D is then the even neighbour) and the
// big flag (a / U >= 2^24: the step leaves the binade).
GE_CHAIN_HD void step_bits(uint32_t ab, int uexp, uint32_t& D, bool& tie, bool& big) {
    uint32_t ma;
    int ea;
    float_fields(ab, ma, ea);
    const int sh = uexp + 150 - ea;  // a / U = ma * 2^-sh
    tie = false;
    big = false;
    D = 0;
    if (ma == 0) return;
    if (sh < 0) {
        big = true;  // ma >= 2^23 here, so a / U >= 2^24
        return;
    }
    if (sh >= 32) return;  // a / U < 2^-8: rounds to 0, no tie
    const uint32_t d0 = ma >> sh;
    if (sh == 0) {
        D = d0;
        return;
    }
    const uint32_t frac = ma & ((1u << sh) - 1u);
    const uint32_t half = 1u << (sh - 1);
    tie = frac == half;
    D = tie ? d0 + (d0 & 1u) : d0 + (frac > half ? 1u : 0u);
}

// Smallest m with m * 2^uexp >= thr, for a float thr; kNoThreshold when thr is
// NaN or unreachable inside the binade (>= 2^(uexp + 24)).
constexpr uint32_t kNoThreshold = 0xFFFFFFFFu;
GE_CHAIN_HD uint32_t threshold_bits(uint32_t tb, int uexp) {
    if ((tb & 0x7FFFFFFFu) > 0x7F800000u) return kNoThreshold;  // NaN
    if ((tb & 0x80000000u) || (tb & 0x7FFFFFFFu) == 0u) return 0u;  // thr <= 0
    if (tb == 0x7F800000u) return kNoThreshold;                    // +inf
    uint32_t mt;
    int et;
    float_fields(tb, mt, et);
    const int d = uexp + 150 - et;  // thr / U = mt * 2^-d
    if (d <= 0) {
        if (d < -8) return kNoThreshold;
        const uint64_t t = static_cast<uint64_t>(mt) << (-d);
        return t >= (1u << 24) ? kNoThreshold : static_cast<uint32_t>(t);
    }
    if (d >= 32) return 1u;
    return (mt >> d) + ((mt & ((1u << d) - 1u)) ? 1u : 0u);
}

// ---- float accumulator, in 32-bit integers --------------------------------
//
// The same two runs for a float accumulator, the case of the top-p
// cumulative and the draw walk. m < 2^24, so the binade arithmetic fits in
// 32-bit integers; the ulp and its inverse come straight from the float's
// exponent field (exact powers of two), and the quotients are 32-bit.

struct BinadeF {
    uint32_t m;     // accumulator / U
    uint32_t lo;    // smallest m a descending step may produce and stay exact
    double ulp;     // U
    double scale;   // 1 / U
};
constexpr uint32_t kHiF = 0xFFFFFFu;  // largest m an ascending step may produce

GE_CHAIN_HD BinadeF binade_f32(double s) {
    const uint32_t sb = __builtin_bit_cast(uint32_t, static_cast<float>(s));
    const uint32_t ex = sb >> 23;
    const bool low = ex <= 1u;  // subnormals and the first normal binade share U = 2^-149
    const int uexp = low ? -149 : static_cast<int>(ex) - 150;
    BinadeF b;
    b.m = low ? (sb & 0x00FFFFFFu) : ((sb & 0x7FFFFFu) | 0x800000u);
    b.lo = low ? 1u : 0x800001u;
    b.ulp = __builtin_bit_cast(double, static_cast<uint64_t>(1023 + uexp) << 52);
    b.scale = __builtin_bit_cast(double, static_cast<uint64_t>(1023 - uexp) << 52);
    return b;
}

GE_CHAIN_HD uint64_t asc_run_f32(double& s, double a, uint64_t n, double thr, bool& hit) {
    hit = false;
    uint64_t done = 0;
    while (done < n) {
        if (!(a > 0.0)) {
            if (s >= thr) {
                hit = true;
                return done + 1;
            }
            return n;
        }
        BinadeF b = binade_f32(s);
        const double A = a * b.scale;
        const double D0 = std::floor(A);
        const double fr = A - D0;
        const uint32_t d0 = A < 16777216.0 ? static_cast<uint32_t>(D0) : 0u;
        const bool tie = fr == 0.5;
        if (s == 0.0 || A >= 16777216.0 || (tie && (b.m & 1u))) {  // one ordinary step
            s = add_once<float>(s, a);
            ++done;
            if (s >= thr) {
                hit = true;
                return done;
            }
            continue;
        }
        const uint32_t D = tie ? d0 + (d0 & 1u) : d0 + (fr > 0.5 ? 1u : 0u);
        const uint64_t rem = n - done;
        const uint64_t jv = D ? (kHiF - b.m) / D : kNone;
        uint64_t jh = kNone;
        if (thr == thr) {
            if (!(thr > 0.0)) {
                jh = 1;
            } else {
                const double tmd = std::ceil(thr * b.scale);
                if (tmd <= 16777216.0) {
                    const uint32_t tm = static_cast<uint32_t>(tmd);
                    if (b.m >= tm) jh = 1;
                    else if (D) jh = (tm - b.m + D - 1) / D;
                }
            }
        }
        uint64_t j = rem < jv ? rem : jv;
        if (jh < j) j = jh;
        b.m += static_cast<uint32_t>(j) * D;
        s = static_cast<double>(b.m) * b.ulp;
        done += j;
        if (j == jh) {
            hit = true;
            return done;
        }
        if (done < n) {
            s = add_once<float>(s, a);
            ++done;
            if (s >= thr) {
                hit = true;
                return done;
            }
        }
    }
    return n;
}

GE_CHAIN_HD uint64_t desc_run_f32(double& c, double a, uint64_t n, bool& stop) {
    stop = false;
    uint64_t done = 0;
    while (done < n) {
        if (c <= a) {
            stop = true;
            return done;
        }
        if (!(a > 0.0)) return n;
        BinadeF b = binade_f32(c);
        const double A = a * b.scale;  // a < c, so A < 2^24
        const double D0 = std::floor(A);
        const double fr = A - D0;
        const uint32_t d0 = static_cast<uint32_t>(D0);
        const bool tie = fr == 0.5;
        if (tie && (b.m & 1u)) {
            c = sub_once<float>(c, a);
            ++done;
            continue;
        }
        const uint32_t D = tie ? d0 + (d0 & 1u) : d0 + (fr > 0.5 ? 1u : 0u);
        if (D == 0 && b.m >= b.lo) return n;
        const uint64_t jv = (D && b.m >= b.lo) ? (b.m - b.lo) / D : 0;
        const uint64_t rem = n - done;
        const uint64_t j = rem < jv ? rem : jv;
        b.m -= static_cast<uint32_t>(j) * D;
        c = static_cast<double>(b.m) * b.ulp;
        done += j;
        if (done < n) {
            if (c <= a) {
                stop = true;
                return done;
            }
            c = sub_once<float>(c, a);
            ++done;
        }
    }
    return n;
}

}  // namespace chain
}  // namespace ge
