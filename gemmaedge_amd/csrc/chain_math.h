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
//
// Written with selects only (no early exits), so a wave evaluating it for
// many addends at once runs no divergent branches:
//   ma == 0      -> D = 0
//   sh < 0       -> big (ma >= 2^23 here, so a / U >= 2^24), D = 0
//   sh >= 32     -> a / U < 2^-8: rounds to 0, no tie
//   0 <= sh < 32 -> D = ma >> sh rounded to nearest by the sh dropped bits
//                   (sh = 0 drops none: frac = half = 0, never a tie).
// odd0 (ties only): floor(a / U) is odd, so D = floor + 1.
GE_CHAIN_HD void step_bits_p(uint32_t ab, int uexp, uint32_t& D, bool& tie, bool& odd0, bool& big) {
    uint32_t ma;
    int ea;
    float_fields(ab, ma, ea);
    const int sh = uexp + 150 - ea;  // a / U = ma * 2^-sh
    const bool nz = ma != 0u;
    const bool in_range = nz && sh >= 0 && sh < 32;
    const uint32_t shc = static_cast<uint32_t>(sh < 0 ? 0 : (sh > 31 ? 31 : sh));
    const uint32_t d0 = ma >> shc;
    const uint32_t frac = ma & ((1u << shc) - 1u);
    const uint32_t half = (1u << shc) >> 1;
    big = nz && sh < 0;
    tie = in_range && shc != 0u && frac == half;
    odd0 = tie && (d0 & 1u) != 0u;
    const uint32_t up = tie ? (d0 & 1u) : (frac > half ? 1u : 0u);
    D = in_range ? d0 + up : 0u;
}
GE_CHAIN_HD void step_bits(uint32_t ab, int uexp, uint32_t& D, bool& tie, bool& big) {
    bool odd0;
    step_bits_p(ab, uexp, D, tie, odd0, big);
}

// The same step for a double accumulator (U = 2^uexp, 53-bit significand)
// and a float addend: D = round(a / U) as a 64-bit integer, big when
// a / U >= 2^53. Addends at or above the ulp are whole multiples of it (no
// rounding); below, as for the float accumulator.
GE_CHAIN_HD void step_bits64(uint32_t ab, int uexp, uint64_t& D, bool& tie, bool& odd0, bool& big) {
    uint32_t ma;
    int ea;
    float_fields(ab, ma, ea);
    const int sh = uexp + 150 - ea;  // a / U = ma * 2^-sh
    D = 0;
    tie = false;
    odd0 = false;
    big = false;
    if (ma == 0u) return;
    if (sh <= 0) {
        const int up = -sh;  // a / U = ma * 2^up, ma < 2^24
        if (up >= 53 || (up >= 30 && ma >= (1u << (53 - up)))) {
            big = true;
            return;
        }
        D = static_cast<uint64_t>(ma) << up;  // < 2^53
        return;
    }
    if (sh >= 32) return;  // a / U < 2^-8
    const uint32_t d0 = ma >> sh;
    const uint32_t frac = ma & ((1u << sh) - 1u);
    const uint32_t half = 1u << (sh - 1);
    tie = frac == half;
    odd0 = tie && (d0 & 1u) != 0u;
    D = d0 + (tie ? (d0 & 1u) : (frac > half ? 1u : 0u));
}

// ---- runs as functions of the accumulator's parity ---------------------------
//
// Inside one binade, a run of n elements of one addend moves m by a fixed
// number of ulps, except that a tie's first element depends on the parity of
// m (ties to even). A run, and any sequence of runs, is therefore the map
// m -> m + e (m even) or m + o (m odd) for ascending sums, m - e / m - o for
// descending ones: two magnitudes. The parity after the map is the start
// parity plus that magnitude, so maps compose associatively and a block of
// threads can scan them; the first element that would leave the binade (or
// reach a threshold) is found from the scanned magnitudes, which only grow
// along the sequence. Magnitudes saturate at kCap, beyond any binade's room.
template <typename U>
struct ParityMap {
    U e;  // magnitude from an even m
    U o;  // magnitude from an odd m
};

template <typename U, U kCap>
GE_CHAIN_HD U sat_add_cap(U x, U y) {
    const U s = x + y;  // x, y <= kCap <= half the range: no wrap
    return s > kCap ? kCap : s;
}

// n elements of one addend with step D (tie / odd0 / big from step_bits*).
// From an odd m a tie's first element moves by D + 1 when floor(a / U) is
// even (D is that floor) and by D - 1 when it is odd (D is floor + 1); m is
// even after it, and every later element moves by D.
template <typename U, U kCap>
GE_CHAIN_HD ParityMap<U> run_map(uint32_t n, U D, bool tie, bool odd0, bool big) {
    ParityMap<U> r{0, 0};
    if (n == 0) return r;
    if (big) {
        r.e = r.o = kCap;
        return r;
    }
    U base;
    if constexpr (sizeof(U) == 4) {  // D <= 2^24 + 1: the product fits 64 bits
        const uint64_t p = static_cast<uint64_t>(n) * D;
        base = p > kCap ? kCap : static_cast<U>(p);
    } else {  // D < 2^53; a product near 2^61 is far beyond any binade's room
        const bool over = static_cast<double>(n) * static_cast<double>(D) >= 2305843009213693952.0;  // 2^61
        base = over ? kCap : static_cast<U>(static_cast<uint64_t>(n) * D);
    }
    r.e = base;
    r.o = (tie && base != kCap) ? (odd0 ? base - 1 : base + 1) : base;
    return r;
}

// f, then g.
template <typename U, U kCap>
GE_CHAIN_HD ParityMap<U> compose(ParityMap<U> f, ParityMap<U> g) {
    ParityMap<U> h;
    h.e = sat_add_cap<U, kCap>(f.e, (f.e & 1u) ? g.o : g.e);
    h.o = sat_add_cap<U, kCap>(f.o, (f.o & 1u) ? g.e : g.o);
    return h;
}

template <typename U>
GE_CHAIN_HD U apply_from(ParityMap<U> f, U m) {
    return (m & 1u) ? f.o : f.e;
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
// cumulative and the draw walk. The accumulator is carried as its float bits:
// binade_bits gives m = accumulator / U, step_bits the per-element increment
// D (with the tie and big flags), threshold_bits the threshold in ulps, and
// the run lengths inside a binade are 32-bit quotients (m < 2^24, D <= 2^24).
// The one element that leaves a binade, and a tie from an odd m, is a plain
// float operation. thr must be a float value (or NaN); s, c >= 0.

GE_CHAIN_HD uint32_t fbits(float x) { return __builtin_bit_cast(uint32_t, x); }
GE_CHAIN_HD float fval(uint32_t b) { return __builtin_bit_cast(float, b); }
// Bits of m * U for an m that stays in the binade of sb.
GE_CHAIN_HD uint32_t rebuild_bits(uint32_t sb, uint32_t m) {
    return (sb >> 23) <= 1u ? m : ((sb & 0x7F800000u) | (m & 0x7FFFFFu));
}
constexpr uint32_t kHiF = 0xFFFFFFu;  // largest m an ascending step may produce

GE_CHAIN_HD uint64_t asc_run_f32(double& s, double a, uint64_t n, double thr, bool& hit) {
    hit = false;
    if (n == 0) return 0;
    if (!(a > 0.0)) {
        if (s >= thr) {
            hit = true;
            return 1;
        }
        return n;
    }
    const float af = static_cast<float>(a);
    const uint32_t ab = fbits(af);
    const uint32_t tb = fbits(static_cast<float>(thr));
    uint32_t sb = fbits(static_cast<float>(s));
    if ((sb & 0x7F800000u) == 0x7F800000u) {  // inf or NaN: no later element changes it
        sb = fbits(fval(sb) + af);
        s = static_cast<double>(fval(sb));
        if (s >= thr) {
            hit = true;
            return 1;
        }
        return n;
    }
    uint64_t done = 0;
    while (done < n) {
        const StepBits b = binade_bits(sb);
        uint32_t D;
        bool tie, big;
        step_bits(ab, b.uexp, D, tie, big);
        if ((sb & 0x7FFFFFFFu) == 0u || big || (tie && (b.m & 1u))) {  // one ordinary step
            sb = fbits(fval(sb) + af);
            ++done;
            if (static_cast<double>(fval(sb)) >= thr) {
                hit = true;
                s = static_cast<double>(fval(sb));
                return done;
            }
            continue;
        }
        const uint64_t rem = n - done;
        // j = min(rem, steps that stay in the binade); the quotient only when
        // the run would leave it (rem * D < 2^57: no wrap)
        const uint32_t room = kHiF - b.m;
        uint64_t j = rem;
        if (D && rem * D > room) j = room / D;  // < rem here
        // steps to reach thr, when that lies within the j steps
        uint64_t jh = kNone;
        const uint32_t tm = threshold_bits(tb, b.uexp);
        if (tm != kNoThreshold) {
            if (b.m >= tm) jh = 1;
            else if (D && b.m + j * D >= tm) jh = (tm - b.m + D - 1u) / D;
        }
        if (jh < j) j = jh;
        sb = rebuild_bits(sb, b.m + static_cast<uint32_t>(j) * D);
        done += j;
        if (j == jh) {
            hit = true;
            s = static_cast<double>(fval(sb));
            return done;
        }
        if (done < n) {
            sb = fbits(fval(sb) + af);
            ++done;
            if (static_cast<double>(fval(sb)) >= thr) {
                hit = true;
                s = static_cast<double>(fval(sb));
                return done;
            }
        }
    }
    s = static_cast<double>(fval(sb));
    return n;
}

GE_CHAIN_HD uint64_t desc_run_f32(double& c, double a, uint64_t n, bool& stop) {
    stop = false;
    if (n == 0) return 0;
    const float af = static_cast<float>(a);
    const uint32_t ab = fbits(af);
    uint32_t cb = fbits(static_cast<float>(c));
    if ((cb & 0x7F800000u) == 0x7F800000u) {  // inf or NaN
        if (fval(cb) <= af) {
            stop = true;
            return 0;
        }
        if (!(a > 0.0)) return n;
        cb = fbits(fval(cb) - af);  // stays inf or NaN
        c = static_cast<double>(fval(cb));
        return n;
    }
    uint64_t done = 0;
    while (done < n) {
        if (fval(cb) <= af) {
            stop = true;
            c = static_cast<double>(fval(cb));
            return done;
        }
        if (!(a > 0.0)) break;
        const StepBits b = binade_bits(cb);
        uint32_t D;
        bool tie, big;
        step_bits(ab, b.uexp, D, tie, big);  // a < c: never big
        if (tie && (b.m & 1u)) {
            cb = fbits(fval(cb) - af);
            ++done;
            continue;
        }
        if (D == 0 && b.m >= b.lo) break;  // every remaining step leaves c unchanged
        // j = min(rem, steps that stay exact in the binade); the quotient only
        // when the run would leave it
        const uint64_t rem = n - done;
        uint64_t j = 0;
        if (D && b.m >= b.lo) j = rem * D <= b.m - b.lo ? rem : (b.m - b.lo) / D;
        cb = rebuild_bits(cb, b.m - static_cast<uint32_t>(j) * D);
        done += j;
        if (done < n) {
            if (fval(cb) <= af) {
                stop = true;
                c = static_cast<double>(fval(cb));
                return done;
            }
            cb = fbits(fval(cb) - af);
            ++done;
        }
    }
    c = static_cast<double>(fval(cb));
    return n;
}

}  // namespace chain
}  // namespace ge
