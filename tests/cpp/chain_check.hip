// Test helper (not part of the product): checks the closed-form replay of
// sequential accumulations (gemmaedge_amd/csrc/chain_math.h) against plain
// left-to-right loops, on the CPU, over random runs built to hit every case:
// binade crossings up and down, ties to even from odd and even starting ulps,
// addends below half an ulp, addends larger than the accumulator, thresholds
// inside, at and beyond a run, and the subnormal region.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <random>
#include <type_traits>
#include <vector>

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

// The 64-bit step of a double accumulator with a float addend against the
// double-based one.
static bool check_step_bits64(std::mt19937_64& g) {
    const int e = static_cast<int>(g() % 120) - 100;
    double s = random_acc<double>(g, e);
    if (g() % 50 == 0) s = 0.0;
    int ea = e - static_cast<int>(g() % 90) + 3;
    if (ea < -149) ea = -149;
    float a = random_float(g, ea, 1 + static_cast<int>(g() % 24));
    if (g() % 50 == 0) a = 0.0f;
    uint32_t ab;
    std::memcpy(&ab, &a, 4);
    const ge::chain::Binade b = ge::chain::binade_of<double>(s);
    const ge::chain::Step st = ge::chain::step_of<double>(b, static_cast<double>(a));
    uint64_t D;
    bool tie, odd0, big;
    ge::chain::step_bits64(ab, b.uexp, D, tie, odd0, big);
    if (st.big != big) return false;
    if (big) return true;
    if (st.D != D || st.tie != tie) return false;
    // odd0: floor(a / U) is odd
    const double A = std::ldexp(static_cast<double>(a), -b.uexp);
    return !tie || odd0 == ((static_cast<uint64_t>(std::floor(A)) & 1u) != 0u);
}

// Host model of the block-wide replay (gemmaedge_amd/csrc/chain_block.h):
// runs are dealt to "threads" of `per` consecutive runs; each thread folds
// its runs' parity maps, the threads' maps are scanned with the same
// doubling pattern as the wave scan (compose(earlier, later) at distances 1,
// 2, 4, ...), and a thread whose scanned magnitude leaves the binade (or
// reaches the threshold) replays its runs to find the first one that does.
// That run is replayed in closed form and the next pass starts after it in
// the new binade. Maps, steps and closed forms are the product's own
// (chain_math.h).
template <bool kF32, bool kDesc>
void block_model(const std::vector<float>& a, const std::vector<uint32_t>& n, int per, double start, double thr,
                 uint64_t& pos, double& s, bool& ev) {
    using U = std::conditional_t<kF32, uint32_t, uint64_t>;
    using Map = ge::chain::ParityMap<U>;
    constexpr U kCap = kF32 ? (1u << 28) : (1ull << 62);
    const size_t runs = a.size();
    const size_t groups = (runs + per - 1) / per;
    std::vector<uint64_t> first(runs + 1, 0);  // first element of each run
    for (size_t i = 0; i < runs; ++i) first[i + 1] = first[i] + n[i];
    s = start;
    size_t it = 0;
    ev = false;
    while (it < runs) {
        U m, lo, hi, tm;
        int uexp;
        if (kF32) {
            float sf = static_cast<float>(s);
            uint32_t sb;
            std::memcpy(&sb, &sf, 4);
            const ge::chain::StepBits b = ge::chain::binade_bits(sb);
            float tf = static_cast<float>(thr);
            uint32_t tb;
            std::memcpy(&tb, &tf, 4);
            m = b.m; lo = b.lo; hi = ge::chain::kHiF; uexp = b.uexp;
            tm = ge::chain::threshold_bits(tb, b.uexp);
        } else {
            const ge::chain::Binade b = ge::chain::binade_of<double>(s);
            m = static_cast<U>(b.m); lo = static_cast<U>(b.lo); hi = static_cast<U>(b.hi); uexp = b.uexp;
            tm = static_cast<U>(~0ull);
            if (thr == thr) {
                if (!(thr > 0.0)) tm = 0;
                else if (thr < std::ldexp(1.0, b.uexp + 53)) tm = static_cast<U>(ge::chain::threshold_m(thr, b.uexp));
            }
        }
        auto exceeds = [&](U r) { return kDesc ? m < lo + r : (m + r > hi || m + r >= tm); };
        auto run_of = [&](size_t i) {  // runs before `it` are consumed: no elements
            uint32_t ab;
            std::memcpy(&ab, &a[i], 4);
            U D;
            bool tie, odd0, big;
            if constexpr (kF32) ge::chain::step_bits_p(ab, uexp, D, tie, odd0, big);
            else ge::chain::step_bits64(ab, uexp, D, tie, odd0, big);
            return ge::chain::run_map<U, kCap>(i >= it ? n[i] : 0u, D, tie, odd0, big);
        };
        std::vector<Map> fold(groups, Map{0, 0});
        for (size_t gi = 0; gi < groups; ++gi)
            for (size_t i = gi * per; i < std::min(runs, (gi + 1) * per); ++i)
                fold[gi] = ge::chain::compose<U, kCap>(fold[gi], run_of(i));
        std::vector<Map> x(groups, Map{0, 0});  // exclusive: shift, then the doubling scan
        for (size_t gi = 1; gi < groups; ++gi) x[gi] = fold[gi - 1];
        for (size_t d = 1; d < groups; d <<= 1) {
            std::vector<Map> y = x;
            for (size_t gi = d; gi < groups; ++gi) y[gi] = ge::chain::compose<U, kCap>(x[gi - d], x[gi]);
            x.swap(y);
        }
        size_t f = runs;
        U r_ev = 0;
        for (size_t gi = 0; gi < groups && f == runs; ++gi) {
            const U r0 = ge::chain::apply_from(x[gi], m);
            const U r_end = ge::chain::sat_add_cap<U, kCap>(r0, ge::chain::apply_from(fold[gi], static_cast<U>(m + r0)));
            if (!exceeds(r_end)) continue;
            U r = r0;
            for (size_t i = gi * per; i < std::min(runs, (gi + 1) * per); ++i) {
                const U rn = ge::chain::sat_add_cap<U, kCap>(r, ge::chain::apply_from(run_of(i), static_cast<U>(m + r)));
                if (i >= it && n[i] && exceeds(rn)) {
                    f = i;
                    r_ev = r;
                    break;
                }
                r = rn;
            }
        }
        auto rebuild = [&](U mm) -> double {
            if (kF32) {
                float sf = static_cast<float>(s);
                uint32_t sb;
                std::memcpy(&sb, &sf, 4);
                const uint32_t nb = ge::chain::rebuild_bits(sb, static_cast<uint32_t>(mm));
                float v;
                std::memcpy(&v, &nb, 4);
                return static_cast<double>(v);
            }
            return std::ldexp(static_cast<double>(mm), uexp);
        };
        if (f == runs) {
            const U rt = groups ? ge::chain::apply_from(ge::chain::compose<U, kCap>(x[groups - 1], fold[groups - 1]), m) : 0;
            s = rebuild(kDesc ? m - rt : m + rt);
            pos = first[runs];
            return;
        }
        double sv = rebuild(kDesc ? m - r_ev : m + r_ev);
        bool hit = false;
        uint64_t used;
        if (kF32) used = kDesc ? ge::chain::desc_run_f32(sv, a[f], n[f], hit) : ge::chain::asc_run_f32(sv, a[f], n[f], thr, hit);
        else used = kDesc ? desc_run<double>(sv, a[f], n[f], hit) : asc_run<double>(sv, a[f], n[f], thr, hit);
        s = sv;
        if (hit) {
            ev = true;
            pos = first[f] + (kDesc ? used : used - 1);
            return;
        }
        it = f + 1;
    }
    pos = first[runs];
}

// Runs as the sorted f32 rows give them: mostly single elements, addends
// descending over many binades, short significands among them (ties).
template <bool kF32, bool kDesc>
bool check_block_model(std::mt19937_64& g) {
    using Acc = std::conditional_t<kF32, float, double>;
    const int runs = 1 + static_cast<int>(g() % 3000);
    std::vector<float> a(runs);
    std::vector<uint32_t> n(runs);
    int e = -static_cast<int>(g() % 8);
    const int drop = 1 + static_cast<int>(g() % 40);  // binades spanned, in 1/64ths per run
    for (int i = 0; i < runs; ++i) {
        if (static_cast<int>(g() % 64) < drop) --e;
        const int bits = (g() % 4 == 0) ? 1 + static_cast<int>(g() % 4) : 1 + static_cast<int>(g() % 24);
        a[i] = random_float(g, e < -140 ? -140 : e, bits);
        if (g() % 200 == 0) a[i] = 0.0f;
        n[i] = (g() % 8 == 0) ? 1 + static_cast<uint32_t>(g() % 5) : 1u;
    }
    std::sort(a.begin(), a.end(), [](float x, float y) { return x > y; });
    double total = 0;
    for (int i = 0; i < runs; ++i) total += static_cast<double>(a[i]) * n[i];
    double start, thr;
    if (kDesc) {
        start = static_cast<double>(static_cast<Acc>(total * (0.01 + (g() % 100) / 100.0)));
        thr = 0.0;
    } else {
        start = static_cast<double>(a[0]);
        thr = kF32 ? static_cast<double>(static_cast<float>(total * (g() % 130) / 100.0)) : std::nan("");
        if (g() % 4 == 0) thr = std::nan("");
    }
    uint64_t pos1;
    double s1;
    bool ev1;
    block_model<kF32, kDesc>(a, n, 1 + static_cast<int>(g() % 8), start, thr, pos1, s1, ev1);
    // every element in order
    Acc v = static_cast<Acc>(start);
    uint64_t pos2 = 0;
    bool ev2 = false;
    for (int i = 0; i < runs && !ev2; ++i) {
        for (uint32_t j = 0; j < n[i]; ++j) {
            if (kDesc) {
                if (static_cast<double>(v) <= static_cast<double>(a[i])) {
                    ev2 = true;
                    break;
                }
                v = v - static_cast<Acc>(a[i]);
            } else {
                v = v + static_cast<Acc>(a[i]);
                if (static_cast<double>(v) >= thr) {
                    ev2 = true;
                    break;
                }
            }
            ++pos2;
        }
    }
    return ev1 == ev2 && pos1 == pos2 && bits_of<Acc>(s1) == bits_of<Acc>(static_cast<double>(v));
}

// which: 0 float asc, 1 float desc, 2 double asc, 3 double desc,
//        4 float asc sequences, 5 float desc sequences, 6 double asc sequences,
//        7 the corrected double quotient,
//        8 / 9 float asc / desc through the 32-bit versions, 10 / 11 their chained runs,
//        12 the bit-field step and threshold of a float accumulator,
//        13 the 64-bit step of a double accumulator,
//        14 / 15 / 16 the block replay's model: float asc / desc, double asc.
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
            case 13: ok = check_step_bits64(g); break;
            case 14: ok = check_block_model<true, false>(g); break;
            case 15: ok = check_block_model<true, true>(g); break;
            case 16: ok = check_block_model<false, false>(g); break;
            default: return -1;
        }
        if (!ok) ++bad;
    }
    return bad;
}
