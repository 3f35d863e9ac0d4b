"""Pins the CPU oracle before it is trusted as the GPU path's checker.

Checks, per oracle function:
  - the reference's own known-answer tests (tests/core_tests.cpp:298-312, :496-500);
  - the reference's own sample_token, built from /root/reference into
    oracle/_ref (tie-free inputs, since the reference's tie order is
    unspecified) — same tokens for the same mt19937_64 stream;
  - the C++ standard's known answer for mt19937_64 ([rand.predef]);
  - closed forms and invariants for the parts the reference lacks or cannot
    pin (penalty, bf16 widening, softcap), and an exact-arithmetic brute force
    on tiny vocabularies for ordering / top-k / top-p / draw.
"""
import math

import numpy as np
import pytest

import ge_oracle as O
from gemmaedge_amd import workloads as W


def sample(values, u=0.5, **kw):
    return O.sample_final(np.asarray(values, np.float32), O.make_params(**kw), u)


# --- reference known answers -------------------------------------------------

def test_core_tests_known_answers():
    # core_tests.cpp:300-304: greedy on {-1, 3, 2} -> 1
    assert sample([-1.0, 3.0, 2.0], temperature=0.0).token == 1
    # core_tests.cpp:306-311: top_k=1, top_p=1, T=1 on {4, 1, 0} -> 0 (for any draw)
    for u in (0.0, 0.3, 0.999):
        assert sample([4.0, 1.0, 0.0], u, temperature=1.0, top_k=1, top_p=1.0).token == 0
    # core_tests.cpp:496-500 relies on first-maximum greedy ties.
    assert sample([1.0] * 5, temperature=0.0).token == 0


def test_empty_logits_rejected():
    with pytest.raises(ValueError):
        O.sample_final(np.zeros(0, np.float32), O.make_params(), 0.5)


# --- RNG and uniform mapping -------------------------------------------------

def test_mt19937_64_standard_known_answer():
    # C++ standard [rand.predef]: the 10000th output of a default-constructed
    # mt19937_64 (seed 5489) is 9981545732273789042.
    assert int(O.mt_outputs(5489, 10000)[-1]) == 9981545732273789042
    e = W.MT19937_64(5489)
    out = [e() for _ in range(10000)]
    assert out[-1] == 9981545732273789042


@pytest.mark.parametrize("seed", [0, 1, 7, 2026, 2**64 - 1])
def test_uniform_mapping_matches_libstdcxx(seed):
    raw = O.mt_outputs(seed, 4096)
    lib = O.mt_uniforms(seed, 4096)  # libstdc++ generate_canonical itself
    restated = np.array([O.uniform_from_u64(int(x)) for x in raw], np.float32)
    python = W.mt_uniforms(seed, 4096)
    assert np.array_equal(restated.view(np.uint32), lib.view(np.uint32))
    assert np.array_equal(python.view(np.uint32), lib.view(np.uint32))


def test_uniform_mapping_edges():
    # float(x)/2^64 rounds up to 1 for x >= 2^64 - 2^39; libstdc++ clamps to nextafter(1, 0).
    below_one = float(np.nextafter(np.float32(1), np.float32(0)))
    for x in (2**64 - 1, 2**64 - 2**39):
        assert O.uniform_from_u64(x) == below_one
        assert W.canonical_float(x) == below_one
    assert O.uniform_from_u64(0) == 0.0
    assert O.uniform_from_u64(2**63) == 0.5
    assert O.uniform_from_u64(2**64 - 2**39 - 1) == float(np.float32(1 - 2**-24))


# --- cross-check against the reference's own sample_token ---------------------

def _distinct_rows(rng, rows, vocab, scale):
    out = np.empty((rows, vocab), np.float32)
    for r in range(rows):
        while True:
            x = (rng.standard_normal(vocab) * scale).astype(np.float32)
            if np.unique(x).size == vocab:
                out[r] = x
                break
    return out


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("cfg", [
    (1.0, 64, 0.95, 0.0), (0.7, 40, 0.9, 0.0), (1.0, 1024, 0.99, 0.0), (1.3, 0, 0.9, 0.0),
    (0.8, 50, 0.8, 0.05), (1.0, 3, 1.0, 0.0), (0.0, 64, 0.9, 0.0), (2.0, 2, 0.0, 0.0),
])
def test_oracle_matches_reference_sample_token(cfg):
    rng = np.random.default_rng(hash(cfg) % 2**32)
    rows, vocab = 120, 3000
    x = _distinct_rows(rng, rows, vocab, 3.0)
    seed = 4242
    ref = O.ref_sample_sequence(x, *cfg, seed)
    u = O.mt_uniforms(seed, rows)
    if cfg[0] <= 0:
        u[:] = 0.0  # greedy consumes no engine output
    out = O.run(x, O.make_params(temperature=cfg[0], top_k=cfg[1], top_p=cfg[2], min_p=cfg[3]),
                uniforms=u)
    assert np.array_equal(out.tokens, ref)


# --- softcap, penalty, bf16 ---------------------------------------------------

def test_softcap_closed_form_and_monotone():
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(20000) * 20, [0.0, -0.0, 1e-30, 500.0, -500.0]])
    x = x.astype(np.float32)
    c = 30.0
    out = O.transform_row(x, O.make_params(softcap=c))
    exact = c * np.tanh(x.astype(np.float64) / c)
    # Division, glibc tanhf (about 2 ulp) and the product round three times:
    # the result stays within 4 float ulps of the exact c * tanh(x / c)
    # (3.34 ulp measured on 200k samples). A dropped term or sign fails this.
    assert np.all(np.abs(out - exact) <= 4 * np.spacing(np.abs(exact).astype(np.float32)) + 1e-45)
    assert np.all(np.abs(out) <= c)
    order = np.argsort(x, kind="stable")
    assert np.all(np.diff(out[order]) >= 0)  # monotone non-decreasing
    # c <= 0 disables it (generation.cpp:431)
    assert np.array_equal(O.transform_row(x, O.make_params(softcap=0.0)), x)


def test_penalty_rule_and_invariants():
    x = np.array([2.0, -2.0, 0.0, 4.0, -0.5, 3.0], np.float32)
    r = 2.0
    out = O.transform_row(x, O.make_params(repetition_penalty=r), history=[0, 1, 2, 2, 2])
    # CTRL rule: positive logits divided, non-positive multiplied, each id once.
    assert out.tolist() == [1.0, -4.0, 0.0, 4.0, -0.5, 3.0]
    # r = 1 is the identity.
    assert np.array_equal(O.transform_row(x, O.make_params(repetition_penalty=1.0), history=[0, 1, 3]), x)
    # duplicates are idempotent, order is irrelevant, out-of-range ids are ignored.
    a = O.transform_row(x, O.make_params(repetition_penalty=1.3), history=[3, 1, 3, 1, 3])
    b = O.transform_row(x, O.make_params(repetition_penalty=1.3), history=[1, 3, -1, 6, 99])
    assert np.array_equal(a, b)
    # applied after the softcap
    c = O.transform_row(x, O.make_params(softcap=30.0, repetition_penalty=2.0), history=[3])
    capped = O.transform_row(x, O.make_params(softcap=30.0))
    assert c[3] == np.float32(capped[3] / np.float32(2.0))


def test_bf16_widening_exact():
    bits = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    bits = bits[((bits.astype(np.uint32) & 0x7F80) != 0x7F80)]  # finite only
    out = O.transform_row(bits, O.make_params())
    assert np.array_equal(out.view(np.uint32), bits.astype(np.uint32) << 16)


# --- softmax / top-p / draw ---------------------------------------------------

def test_softmax_properties():
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(5000) * 3).astype(np.float32)
    r = sample(x, 0.4, temperature=0.8, top_k=200, top_p=2.0)
    assert r.k == 200 and r.keep == 200       # top_p > 1: nothing stops the scan
    assert abs(r.mass - 1.0) < 1e-5            # normalised over the top-k
    top = np.sort(x)[::-1][:200].astype(np.float64)
    p = np.exp((top - top[0]) / 0.8)
    assert abs(r.denominator - p.sum()) / p.sum() < 1e-6


def test_top_p_keeps_at_least_two():
    # generation.cpp:109: the top-p stop needs keep > 0, so a dominant first
    # token still keeps two candidates.
    r = sample([10.0, 0.0, -1.0], 0.99999, temperature=1.0, top_k=3, top_p=0.5)
    assert r.keep == 2
    r = sample([10.0, 0.0, -1.0], 0.5, temperature=1.0, top_k=3, top_p=0.0)
    assert r.keep == 2
    r = sample([10.0, 0.0, -1.0], 0.5, temperature=1.0, top_k=1, top_p=0.0)
    assert r.keep == 1


def test_min_p_cut():
    v = np.log(np.array([0.5, 0.3, 0.1, 0.06, 0.04], np.float64)).astype(np.float32)
    r = sample(v, 0.5, temperature=1.0, top_k=5, top_p=2.0, min_p=0.15)
    assert r.keep == 3   # 0.06 < 0.15 * 0.5


def test_draw_extremes():
    v = np.array([3.0, 2.0, 1.0, 0.0], np.float32)
    assert sample(v, 0.0, temperature=1.0, top_k=4, top_p=2.0).position == 0
    last = sample(v, float(np.nextafter(np.float32(1), np.float32(0))), temperature=1.0, top_k=4,
                  top_p=2.0)
    assert last.position == 3


def test_brute_force_tiny_vocab():
    """Independent formulation in exact (double) arithmetic: full sort by
    (value desc, index asc), softmax over k, top-p / min-p cut and the CDF
    interval containing u * mass. Must agree except for draws within 1e-6 of a
    boundary (reported by the oracle's flag)."""
    rng = np.random.default_rng(99)
    checked = 0
    for _ in range(3000):
        V = int(rng.integers(1, 7))
        vals = rng.integers(-3, 4, size=V).astype(np.float32) * np.float32(rng.choice([0.5, 1.0, 1.7]))
        T = float(rng.choice([0.5, 1.0, 2.0]))
        k = int(rng.integers(0, V + 2))
        top_p = float(rng.choice([0.3, 0.6, 0.9, 1.0]))
        min_p = float(rng.choice([0.0, 0.2]))
        u = float(np.float32(rng.random()))
        r = sample(vals, u, temperature=T, top_k=k, top_p=top_p, min_p=min_p)
        order = sorted(range(V), key=lambda i: (-float(vals[i]), i))
        kk = min(k, V) if k else V
        order = order[:kk]
        m = float(vals[order[0]])
        e = [math.exp((float(vals[i]) - m) / T) for i in order]
        s = sum(e)
        p = [x / s for x in e]
        keep, cum = 0, 0.0
        while keep < kk:
            if p[keep] < p[0] * min_p and keep > 0:
                break
            cum += p[keep]
            if cum >= top_p and keep > 0:
                keep += 1
                break
            keep += 1
        keep = max(keep, 1)
        mass = sum(p[:keep])
        draw = u * mass
        acc, pos = 0.0, keep - 1
        for i in range(keep):
            acc += p[i]
            if draw <= acc:
                pos = i
                break
        if r.near_boundary:
            continue
        # fp32 vs exact arithmetic may move a cut that sits exactly on top_p
        if any(abs(sum(p[:j + 1]) - top_p) < 1e-5 for j in range(kk)):
            continue
        assert r.keep == keep
        assert r.token == order[pos], (vals, T, k, top_p, min_p, u)
        checked += 1
    assert checked > 1500
