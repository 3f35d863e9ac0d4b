// Test helper (not part of the product): checks the closed-form replay of
// sequential accumulations (gemmaedge_amd/csrc/chain_math.h) against plain
// left-to-right loops, on the CPU, over random runs built to hit every case:
// binade crossings up and down, ties to even from odd and even starting ulps,
// addends below half an ulp, addends larger than the accumulator, thresholds
// inside, at and beyond a run, and the subnormal region.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <random>

#include "../../gemmaedge_amd/csrc/chain_math.h"

#pragma clang fp contract(off)

namespace {

using ge::chain::asc_run;
using ge::chain::desc_run;

template <typename Acc>
uint64_t bits_of(double v) {
    if constexpr (sizeof(Acc) == 4) {
        float f = static_cast<float>(v);
        uint32_t b;
        std::memcpy(&b, &f, 4);
        return b;
    } else {
        uint64_t b;
        std::memcpy(&b, &v, 8);
        return b;
    }
}

// A float with `bits` significant bits and exponent e (value in [2^e, 2^(e+1))).
float random_float(std::mt19937_64& g, int e, int bits) {
    if (bits < 1) bits = 1;
    if (bits > 24) bits = 24;
    uint64_t man = (g() & ((1ull << (bits - 1)) - 1)) | (1ull << (bits - 1));
    return static_cast<float>(std::ldexp(static_cast<double>(man), e - (bits - 1)));
}

template <typename Acc>
Acc random_acc(std::mt19937_64& g, int e) {
    if constexpr (sizeof(Acc) == 4) {
        return random_float(g, e, 1 + static_cast<int>(g() % 24));
    } else {
        const int bits = 1 + static_cast<int>(g() % 53);
        uint64_t man = (g() & ((1ull << (bits - 1)) - 1)) | (1ull << (bits - 1));
        return std::ldexp(static_cast<double>(man), e - (bits - 1));
    }
}

struct Case {
    double s;
    double a;
    uint64_t n;
    double thr;
};

template <typename Acc>
Case make_case(std::mt19937_64& g, bool desc) {
    Case c{};
    const int emin = sizeof(Acc) == 4 ? -148 : -1070;
    int e = static_cast<int>(g() % 40) - 30;
    if (g() % 16 == 0) e = emin + static_cast<int>(g() % 6);  // subnormal region
    c.s = (g() % 32 == 0 && !desc) ? 0.0 : static_cast<double>(random_acc<Acc>(g, e));
    // Addend: a few binades below the accumulator, short significands make ties.
    int ea = e - static_cast<int>(g() % 30);
    if (g() % 8 == 0) ea = e + static_cast<int>(g() % 3);
    if (ea < -149) ea = -149;
    c.a = static_cast<double>(random_float(g, ea, 1 + static_cast<int>(g() % 24)));
    if (g() % 40 == 0) c.a = 0.0;
    const int lg = static_cast<int>(g() % 16);
    c.n = 1 + (g() % (1ull << lg));
    c.thr = std::nan("");
    if (!desc) {
        switch (g() % 6) {
            case 0: case 1: break;  // no threshold
            case 2: c.thr = c.s + c.a * static_cast<double>(g() % (c.n + 2)); break;
            case 3: c.thr = -1.0; break;
            case 4: c.thr = static_cast<float>(c.s + c.a * static_cast<double>(c.n) * 0.5); break;
            default: c.thr = static_cast<float>(c.s * (1.0 + static_cast<double>(g() % 100) / 50.0)); break;
        }
        if (c.thr == c.thr) c.thr = static_cast<double>(static_cast<float>(c.thr));
    }
    return c;
}

template <typename Acc, bool kF32 = false>
bool check_asc(const Case& c) {
    double s1 = c.s;
    bool hit1 = false;
    const uint64_t k1 = kF32 ? ge::chain::asc_run_f32(s1, c.a, c.n, c.thr, hit1)
                             : asc_run<Acc>(s1, c.a, c.n, c.thr, hit1);
    Acc s = static_cast<Acc>(c.s);
    uint64_t k2 = c.n;
    bool hit2 = false;
    for (uint64_t i = 0; i < c.n; ++i) {
        s = s + static_cast<Acc>(c.a);
        if (static_cast<double>(s) >= c.thr) {
            hit2 = true;
            k2 = i + 1;
            break;
        }
    }
    return k1 == k2 && hit1 == hit2 && bits_of<Acc>(s1) == bits_of<Acc>(static_cast<double>(s));
}

template <typename Acc, bool kF32 = false>
bool check_desc(const Case& c) {
    double c1 = c.s;
    bool stop1 = false;
    const uint64_t k1 = kF32 ? ge::chain::desc_run_f32(c1, c.a, c.n, stop1) : desc_run<Acc>(c1, c.a, c.n, stop1);
    Acc v = static_cast<Acc>(c.s);
    uint64_t k2 = c.n;
    bool stop2 = false;
    for (uint64_t i = 0; i < c.n; ++i) {
        if (static_cast<double>(v) <= c.a) {
            stop2 = true;
            k2 = i;
            break;
        }
        v = v - static_cast<Acc>(c.a);
    }
    return k1 == k2 && stop1 == stop2 && bits_of<Acc>(c1) == bits_of<Acc>(static_cast<double>(v));
}

// A chain of runs with descending addends (as sorted probabilities are),
// replayed run by run, against one loop over every element.
template <typename Acc, bool kDesc, bool kF32 = false>
bool check_sequence(std::mt19937_64& g) {
    const int runs = 1 + static_cast<int>(g() % 200);
    std::vector<double> a(runs);
    std::vector<uint64_t> n(runs);
    int e = -static_cast<int>(g() % 20);
    for (int i = 0; i < runs; ++i) {
        e -= static_cast<int>(g() % 2);
        a[i] = static_cast<double>(random_float(g, e, 4 + static_cast<int>(g() % 21)));
        n[i] = 1 + g() % 400;
    }
    double total = 0;
    for (int i = 0; i < runs; ++i) total += a[i] * static_cast<double>(n[i]);
    const double start = kDesc ? static_cast<double>(static_cast<Acc>(total * (0.05 + (g() % 100) / 100.0)))
                               : 0.0;
    const double thr = kDesc ? 0.0 : static_cast<double>(static_cast<float>(total * (g() % 120) / 100.0));
    // closed form
    double s1 = start;
    uint64_t pos1 = 0;
    bool ev1 = false;
    for (int i = 0; i < runs && !ev1; ++i) {
        bool ev = false;
        uint64_t k;
        if (kF32) k = kDesc ? ge::chain::desc_run_f32(s1, a[i], n[i], ev) : ge::chain::asc_run_f32(s1, a[i], n[i], thr, ev);
        else k = kDesc ? desc_run<Acc>(s1, a[i], n[i], ev) : asc_run<Acc>(s1, a[i], n[i], thr, ev);
        pos1 += k;
        ev1 = ev;
    }
    // loop
    Acc s = static_cast<Acc>(start);
    uint64_t pos2 = 0;
    bool ev2 = false;
    for (int i = 0; i < runs && !ev2; ++i) {
        for (uint64_t j = 0; j < n[i]; ++j) {
            if (kDesc) {
                if (static_cast<double>(s) <= a[i]) {
                    ev2 = true;
                    break;
                }
                s = s - static_cast<Acc>(a[i]);
                ++pos2;
            } else {
                s = s + static_cast<Acc>(a[i]);
                ++pos2;
                if (static_cast<double>(s) >= thr) {
                    ev2 = true;
                    break;
                }
            }
        }
    }
    return pos1 == pos2 && ev1 == ev2 && bits_of<Acc>(s1) == bits_of<Acc>(static_cast<double>(s));
}

}  // namespace

static bool check_udiv(std::mt19937_64& g) {
    const uint64_t a = g() >> (10 + g() % 54);  // below 2^54
    uint64_t b = g() >> (g() % 64);
    if (b == 0) b = 1;
    return ge::chain::udiv(a, b) == a / b;
}

// The bit-field step of a float accumulator against the double-based one.
static bool check_step_bits(std::mt19937_64& g) {
    const int e = static_cast<int>(g() % 60) - 50;
    float s = random_float(g, (g() % 16 == 0) ? -149 + static_cast<int>(g() % 4) : e, 1 + static_cast<int>(g() % 24));
    if (g() % 50 == 0) s = 0.0f;
    int ea = e - static_cast<int>(g() % 40) + 3;
    if (ea < -149) ea = -149;
    float a = random_float(g, ea, 1 + static_cast<int>(g() % 24));
    if (g() % 50 == 0) a = 0.0f;
    uint32_t sb, ab;
    std::memcpy(&sb, &s, 4);
    std::memcpy(&ab, &a, 4);
    const ge::chain::Binade b1 = ge::chain::binade_of<float>(static_cast<double>(s));
    const ge::chain::StepBits b2 = ge::chain::binade_bits(sb);
    if (b1.m != b2.m || b1.lo != b2.lo || b1.uexp != b2.uexp) return false;
    const ge::chain::Step st = ge::chain::step_of<float>(b1, static_cast<double>(a));
    uint32_t D;
    bool tie, big;
    ge::chain::step_bits(ab, b2.uexp, D, tie, big);
    if (st.big != big) return false;
    if (!big && (st.D != D || st.tie != tie)) return false;
    // threshold in ulps
    float thr = random_float(g, e + static_cast<int>(g() % 6) - 3, 1 + static_cast<int>(g() % 24));
    switch (g() % 10) {
        case 0: thr = -thr; break;
        case 1: thr = 0.0f; break;
        case 2: thr = std::nanf(""); break;
        case 3: thr = INFINITY; break;
        default: break;
    }
    uint32_t tb;
    std::memcpy(&tb, &thr, 4);
    const uint32_t tm = ge::chain::threshold_bits(tb, b2.uexp);
    uint64_t want;
    if (thr != thr || thr == INFINITY) want = ge::chain::kNoThreshold;
    else if (!(thr > 0.0f)) want = 0;
    else {
        const double td = std::ceil(std::ldexp(static_cast<double>(thr), -b2.uexp));
        want = td >= 16777216.0 ? ge::chain::kNoThreshold : static_cast<uint64_t>(td);
    }
    return tm == want;
}

// which: 0 float asc, 1 float desc, 2 double asc, 3 double desc,
//        4 float asc sequences, 5 float desc sequences, 6 double asc sequences,
//        7 the corrected double quotient,
//        8 / 9 float asc / desc through the 32-bit versions, 10 / 11 their chained runs,
//        12 the bit-field step and threshold of a float accumulator.
// Returns the number of mismatching trials (or -1 for a bad `which`).
extern "C" long long ge_test_chain_random(int which, unsigned long long seed, int trials) {
    std::mt19937_64 g(seed);
    long long bad = 0;
    for (int t = 0; t < trials; ++t) {
        bool ok = true;
        switch (which) {
            case 0: ok = check_asc<float>(make_case<float>(g, false)); break;
            case 1: ok = check_desc<float>(make_case<float>(g, true)); break;
            case 2: ok = check_asc<double>(make_case<double>(g, false)); break;
            case 3: ok = check_desc<double>(make_case<double>(g, true)); break;
            case 4: ok = check_sequence<float, false>(g); break;
            case 5: ok = check_sequence<float, true>(g); break;
            case 6: ok = check_sequence<double, false>(g); break;
            case 7: ok = check_udiv(g); break;
            case 8: ok = check_asc<float, true>(make_case<float>(g, false)); break;
            case 9: ok = check_desc<float, true>(make_case<float>(g, true)); break;
            case 10: ok = check_sequence<float, false, true>(g); break;
            case 11: ok = check_sequence<float, true, true>(g); break;
            case 12: ok = check_step_bits(g); break;
            default: return -1;
        }
        if (!ok) ++bad;
    }
    return bad;
}
