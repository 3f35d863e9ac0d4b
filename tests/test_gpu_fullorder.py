"""GPU parity of the full-order path: bf16 rows whose top-k is disabled or
above the selection path's limit (src/generation.cpp:80, k = V when top_k is
0), sampled by the histogram + exact-chain kernels, against the CPU oracle
(a full sort and the reference's sequential sums). Tokens and probabilities
must be bit-identical and the near-boundary flags must agree."""
import numpy as np
import pytest

import ge_oracle as O
from gemmaedge_amd import workloads as W
from gpu_util import assert_parity, run_gpu, run_oracle, small_workload

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sampler():
    import torch

    from gemmaedge_amd import Sampler, available

    assert torch.cuda.is_available(), "GPU test run without a GPU"
    assert available(), "no gfx950 device visible to the HIP library"
    s = Sampler(max_rows=512, max_vocab=W.VOCAB, max_history=20000)
    yield s
    s.close()


def _check(sampler, w, label=""):
    print(f"[fullorder] {label or w.name} rows={w.rows} V={w.vocab} {w.dtype} {w.params}", flush=True)
    gpu = run_gpu(sampler, w)
    ora = run_oracle(w)
    assert_parity(w, gpu, ora, label)
    return gpu, ora


def _bf16(x):
    return W.f32_to_bf16_bits(np.asarray(x, np.float32))


def test_c4_rows(sampler):
    gpu, ora = _check(sampler, W.c4(rows=48))
    assert np.all(ora.results["k"] == W.VOCAB)
    assert np.all(ora.results["keep"] > 200000)  # a nucleus of ~232k tokens


def test_wide_range_rows_replay_the_double_denominator(sampler):
    # N(0, 3) logits: probabilities span ~30 binades, so the double
    # denominator is not exact in every order and is replayed in closed form;
    # top_p = 1 with u near 1 walks deep into the tail.
    rng = np.random.default_rng(21)
    x = (rng.standard_normal((6, W.VOCAB)) * 3).astype(np.float32)
    u = np.array([0.5, 0.999, 0.99999, 0.0, 0.25, float(np.float32(1 - 2**-24))], np.float32)
    for top_p in (0.9, 1.0, 2.0):
        w = small_workload(f"wide-p{top_p}", _bf16(x), dict(temperature=1.0, top_k=0, top_p=top_p, softcap=30.0),
                           uniforms=u, dtype="bf16")
        _check(sampler, w)


def test_special_values(sampler):
    rng = np.random.default_rng(3)
    V = 5003
    base = (rng.standard_normal(V) * 0.5).astype(np.float32)
    rows = []
    r = base.copy(); r[::97] = np.nan; rows.append(r)                     # NaNs inside the top-k
    r = base.copy(); r[5] = np.inf; r[9] = -np.inf; rows.append(r)         # +inf max
    r = base.copy(); r[::3] = 0.0; r[1::3] = -0.0; rows.append(r)          # +-0 ties
    r = np.zeros(V, np.float32); rows.append(r)                            # one value
    r = np.full(V, np.nan, np.float32); rows.append(r)                     # all NaN
    r = base.copy(); r[:] = -np.inf; r[100] = 1.0; rows.append(r)          # -inf tail
    x = _bf16(np.stack(rows))
    for T in (1.0, 0.3):
        for cap in (0.0, 30.0):
            for k in (0, 2000):
                w = small_workload(f"special-T{T}-c{cap}-k{k}", x,
                                   dict(temperature=T, top_k=k, top_p=0.9, softcap=cap),
                                   uniforms=W.mt_uniforms(int(T * 10 + cap + k), x.shape[0]), dtype="bf16")
                _check(sampler, w)


def test_degenerate_temperatures(sampler):
    rng = np.random.default_rng(4)
    x = _bf16(rng.standard_normal((3, 3000)).astype(np.float32))
    for T in (1e-30, float("nan"), float("inf"), 1e30):
        w = small_workload(f"T{T}", x, dict(temperature=T, top_k=0, top_p=0.9), dtype="bf16")
        _check(sampler, w)


def test_penalties(sampler):
    rng = np.random.default_rng(5)
    V = 8192
    x = (rng.standard_normal((4, V)) * 2).astype(np.float32)
    x[0, :50] = 0.0
    x[1, 10] = np.nan
    x[2, :] = np.round(x[2, :])  # heavy ties before and after the penalty
    xb = _bf16(x)
    H = 3000
    hist = rng.integers(-5, V + 5, size=4 * H).astype(np.int32)  # duplicates and out-of-range ids
    hist[:50] = np.arange(50)  # row 0: the zeros are penalised
    hist[H + 7] = 10           # row 1: a NaN token is penalised
    offs = (np.arange(5) * H).astype(np.int32)
    for r in (1.3, 0.7, 1.0):
        for cap in (0.0, 30.0):
            w = small_workload(f"pen-r{r}-c{cap}", xb,
                               dict(temperature=0.9, top_k=0, top_p=0.95, softcap=cap, repetition_penalty=r),
                               history=hist, offsets=offs, uniforms=W.mt_uniforms(int(r * 100 + cap), 4),
                               dtype="bf16")
            _check(sampler, w)


def test_k_truncates_inside_a_tie_group(sampler):
    rng = np.random.default_rng(6)
    V = 4099  # not a multiple of 8: scalar tail
    x = _bf16(rng.integers(-4, 5, size=(5, V)).astype(np.float32))
    for k in (1025, 1500, 3000, 4098, 4099, 10**6):
        for min_p in (0.0, 0.3, 0.9, 1.5):
            w = small_workload(f"k{k}-minp{min_p}", x,
                               dict(temperature=0.8, top_k=k, top_p=0.9, min_p=min_p),
                               uniforms=W.mt_uniforms(k % 1000 + int(min_p * 10), 5), dtype="bf16")
            _check(sampler, w)


def test_top_p_edges(sampler):
    rng = np.random.default_rng(7)
    x = _bf16((rng.standard_normal((4, 20000)) * 0.2).astype(np.float32))
    for top_p in (0.0, 0.5, 0.999, 1.0, 2.0, float("nan"), -1.0):
        w = small_workload(f"p{top_p}", x, dict(temperature=1.3, top_k=0, top_p=top_p, softcap=30.0),
                           dtype="bf16")
        _check(sampler, w)


def test_unaligned_rows(sampler):
    import torch

    from gemmaedge_amd import SamplingConfig

    rng = np.random.default_rng(8)
    x = _bf16((rng.standard_normal((3, 5000)) * 0.3).astype(np.float32))
    flat = torch.from_numpy(np.concatenate([[0], x.ravel()]).astype(np.uint16).view(np.int16)).cuda()
    logits = flat[1:].view(torch.bfloat16).view(3, 5000)  # 2-byte offset: no 16-byte loads
    uni = W.mt_uniforms(9, 3)
    cfg = SamplingConfig(temperature=1.0, top_k=0, top_p=0.9, softcap=30.0)
    tokens, probs, _ = sampler.sample(logits, cfg, uniforms=torch.from_numpy(uni).cuda())
    torch.cuda.synchronize()
    ora = O.run(x, O.make_params(temperature=1.0, top_k=0, top_p=0.9, softcap=30.0), uniforms=uni)
    assert np.array_equal(tokens.cpu().numpy(), ora.tokens)
    assert np.array_equal(probs.cpu().numpy().view(np.uint32), ora.probs.view(np.uint32))


def test_random_cases(sampler):
    rng = np.random.default_rng(2024)
    for case in range(60):
        V = int(rng.choice([1025, 1500, 4096, 4099, 20000, 70001]))
        rows = int(rng.integers(1, 4))
        kind = rng.integers(0, 4)
        if kind == 0:
            x = rng.standard_normal((rows, V)) * rng.uniform(0.05, 4)
        elif kind == 1:
            x = rng.integers(-3, 4, size=(rows, V)).astype(np.float64)
        elif kind == 2:
            x = rng.standard_normal((rows, V)) * 200
        else:
            x = rng.choice(np.array([0.0, -0.0, 1e-30, 2.0, -1.0]), size=(rows, V))
        params = dict(temperature=float(rng.choice([0.5, 1.0, 1.7])),
                      top_k=int(rng.choice([0, 0, 1025, 3000])),
                      top_p=float(rng.choice([0.0, 0.5, 0.9, 0.95, 1.0, 1.5])),
                      min_p=float(rng.choice([0.0, 0.0, 0.05, 0.5])),
                      softcap=float(rng.choice([0.0, 30.0, 5.0])),
                      repetition_penalty=float(rng.choice([1.0, 1.1, 1.5, 0.8])))
        H = int(rng.choice([0, 1, 7, 64, 300]))
        hist = rng.integers(-2, V + 2, size=rows * H).astype(np.int32)
        offsets = (np.arange(rows + 1) * H).astype(np.int32)
        w = small_workload(f"fo-rand{case}", _bf16(x), params, hist, offsets, W.mt_uniforms(case, rows),
                           dtype="bf16")
        _check(sampler, w)


def test_per_row_params_mix_paths(sampler):
    import torch

    from gemmaedge_amd import SamplingConfig

    rng = np.random.default_rng(10)
    rows, V = 6, 30000
    x = _bf16((rng.standard_normal((rows, V)) * 1.5).astype(np.float32))
    cfgs = [SamplingConfig(temperature=t, top_k=k, top_p=p, softcap=30.0, repetition_penalty=1.1)
            for t, k, p in [(0.0, 0, 0.9), (1.0, 0, 0.95), (0.7, 40, 0.9), (1.0, 5000, 0.99),
                            (1.2, 1024, 1.0), (0.5, 1025, 0.5)]]
    hist = rng.integers(0, V, size=rows * 32).astype(np.int32)
    offs = (np.arange(rows + 1) * 32).astype(np.int32)
    uni = W.mt_uniforms(12, rows)
    xt = torch.from_numpy(x.view(np.int16)).cuda().view(torch.bfloat16)
    tokens, probs, flags = sampler.sample(
        xt, cfgs, uniforms=torch.from_numpy(uni).cuda(),
        history=torch.from_numpy(hist).cuda(), history_offsets=torch.from_numpy(offs).cuda())
    torch.cuda.synchronize()
    params = [O.make_params(temperature=c.temperature, top_k=c.top_k, top_p=c.top_p,
                            softcap=c.softcap, repetition_penalty=c.repetition_penalty) for c in cfgs]
    ora = O.run(x, params, history=hist, offsets=offs, uniforms=uni)
    assert np.array_equal(tokens.cpu().numpy(), ora.tokens)
    assert np.array_equal(probs.cpu().numpy().view(np.uint32), ora.probs.view(np.uint32))
    assert np.array_equal(flags.cpu().numpy() & 1, ora.flags)


def test_more_penalised_tokens_than_extras(sampler):
    # 9000 unique history ids exceed the histogram pass's 8192 extras: the
    # row is re-sampled by the fallback pass (sorted items, as for f32 rows)
    # and matches the oracle; nothing is flagged unsupported.
    from gemmaedge_amd import sampler as S

    rng = np.random.default_rng(11)
    V = 40000
    x = _bf16(rng.standard_normal((1, V)).astype(np.float32))
    hist = rng.permutation(V)[:9000].astype(np.int32)  # 9000 unique ids > 8192
    w = small_workload("many-penalised", x, dict(temperature=1.0, top_k=0, repetition_penalty=1.2),
                       history=hist, offsets=np.array([0, hist.size], np.int32), dtype="bf16")
    gpu, _ = _check(sampler, w)
    assert not (gpu[2][0] & S.GE_FLAG_UNSUPPORTED)
    # the history bitmap was restored: the next call on the same rows is exact
    w2 = small_workload("after-many", x, dict(temperature=1.0, top_k=0, repetition_penalty=1.2),
                        history=hist[:100], offsets=np.array([0, 100], np.int32), dtype="bf16")
    _check(sampler, w2)


def test_penalised_overflow_rows_in_slices():
    # A handle whose workspace holds one f32-stride row at a time: the
    # fallback pass runs three slices. Rows 0 and 2 overflow the extras (10000
    # unique ids), row 1 does not and keeps the first pass's result; row 2
    # with penalty below 1.
    import torch

    from gemmaedge_amd import Sampler
    from gemmaedge_amd import sampler as S

    rng = np.random.default_rng(12)
    V = W.VOCAB
    x = _bf16((rng.standard_normal((3, V)) * 0.5).astype(np.float32))
    lens = [10000, 300, 10000]
    hist = np.concatenate([rng.permutation(V)[:n] for n in lens]).astype(np.int32)
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    for r in (1.3, 0.85):
        w = small_workload(f"overflow-slices-r{r}", x, dict(temperature=1.0, top_k=0, top_p=0.95,
                                                           softcap=30.0, repetition_penalty=r),
                           history=hist, offsets=offs, uniforms=W.mt_uniforms(77, 3), dtype="bf16")
        s = Sampler(max_rows=4, max_vocab=V, max_history=12000)
        try:
            gpu = run_gpu(s, w)
            torch.cuda.synchronize()
        finally:
            s.close()
        ora = run_oracle(w)
        assert_parity(w, gpu, ora, w.name)
        assert not np.any(gpu[2] & S.GE_FLAG_UNSUPPORTED), gpu[2]


def test_values_with_more_than_32768_tokens(sampler):
    """Bins whose count passes the LDS counters' 16-bit fields (moved to the
    spill list every 32768 tokens), including one whose remaining field is
    exactly 0 and a NaN bin that spills."""
    V = 100003
    rng = np.random.default_rng(21)
    base = (rng.standard_normal(V) * 0.5).astype(np.float32)
    rows = [np.zeros(V, np.float32)]                                         # one value, 3 spills
    r = base.copy(); r[: 2 * 32768] = 0.25; rows.append(r)                   # field 0 after 2 spills
    r = base.copy(); r[5:5 + 32768] = -1.5; r[40000:40000 + 40000] = np.nan; rows.append(r)
    r = base.copy(); r[::2] = -np.inf; rows.append(r)                         # -inf bin with 50002 tokens
    r = np.full(V, 0.125, np.float32); r[7::3] = 0.5; rows.append(r)          # two heavy values
    x = _bf16(np.stack(rows))
    for T, p in ((1.0, 0.9), (0.7, 1.0)):
        w = small_workload(f"spill-T{T}-p{p}", x, dict(temperature=T, top_k=0, top_p=p, softcap=30.0),
                           uniforms=W.mt_uniforms(int(T * 10), x.shape[0]), dtype="bf16")
        _check(sampler, w)


def test_scan_skips_batches_by_speculative_counts(sampler):
    """bf16 rows of many token-scan batches (16384 tokens each) where the
    draw lands where the decide kernel's idle waves predicted, so the token
    scan starts at a later batch from their per-batch counts: narrow N(0, 0.1)
    rows (every group near the draw is counted), a vocabulary whose last batch
    is partial, penalised ids inside the counted batches (the bitmap masks
    them and the extras run adds those of the selected value back), heavy ties
    (groups of thousands of tokens, penalised ones among them), cuts that end
    the mass early (min-p, top-p) and draws at both ends (u = 0, u -> 1)."""
    rng = np.random.default_rng(31)
    u_edge = np.array([0.0, float(np.float32(1 - 2**-24)), 0.5, 0.25, 0.75, 0.999], np.float32)
    for V in (W.VOCAB, 100003):
        x = (rng.standard_normal((6, V)) * 0.1).astype(np.float32)
        x[3] = np.round(x[3] * 40) / 40  # ~30 distinct values
        xb = _bf16(x)
        H = 2000
        hist = rng.integers(0, V, size=6 * H).astype(np.int32)
        offs = (np.arange(7) * H).astype(np.int32)
        for pen in (1.0, 1.3, 0.8):
            for top_p, min_p in ((0.9, 0.0), (1.0, 0.0), (0.95, 0.5), (0.3, 0.0)):
                for uni in (W.mt_uniforms(int(pen * 10) + int(top_p * 100) + V % 7, 6), u_edge):
                    w = small_workload(f"spec-V{V}-r{pen}-p{top_p}-m{min_p}", xb,
                                       dict(temperature=1.3, top_k=0, top_p=top_p, min_p=min_p, softcap=30.0,
                                            repetition_penalty=pen),
                                       history=hist, offsets=offs, uniforms=uni, dtype="bf16")
                    _check(sampler, w)


def test_scan_skips_batches_on_unaligned_rows(sampler):
    # a 2-byte row offset: the counting waves and the scan take scalar loads
    import torch

    from gemmaedge_amd import SamplingConfig

    rng = np.random.default_rng(32)
    V = 70001
    x = _bf16((rng.standard_normal((4, V)) * 0.1).astype(np.float32))
    flat = torch.from_numpy(np.concatenate([[0], x.ravel()]).astype(np.uint16).view(np.int16)).cuda()
    logits = flat[1:].view(torch.bfloat16).view(4, V)
    hist = rng.integers(0, V, size=4 * 500).astype(np.int32)
    offs = (np.arange(5) * 500).astype(np.int32)
    uni = W.mt_uniforms(33, 4)
    cfg = SamplingConfig(temperature=1.3, top_k=0, top_p=0.9, softcap=30.0, repetition_penalty=1.2)
    tokens, probs, _ = sampler.sample(logits, cfg, uniforms=torch.from_numpy(uni).cuda(),
                                      history=torch.from_numpy(hist).cuda(),
                                      history_offsets=torch.from_numpy(offs).cuda())
    torch.cuda.synchronize()
    ora = O.run(x, O.make_params(temperature=1.3, top_k=0, top_p=0.9, softcap=30.0, repetition_penalty=1.2),
                history=hist, offsets=offs, uniforms=uni)
    assert np.array_equal(tokens.cpu().numpy(), ora.tokens)
    assert np.array_equal(probs.cpu().numpy().view(np.uint32), ora.probs.view(np.uint32))


def test_top_p_chain_passes_segments_by_their_totals(sampler):
    """The top-p chain of bf16 rows passes 128-item segments of its last binade
    by totals the idle waves wrote while it ran the binades below. Thresholds
    at and near binade edges (the table's binade is that of top_p), sharp and
    flat rows (few or many items in that binade), ties, penalised ids and a
    min-p cut that ends the chain inside the table's segments."""
    rng = np.random.default_rng(41)
    V = 70001
    rows = []
    for sd in (0.05, 0.1, 0.3, 1.0):
        rows.append(rng.standard_normal(V) * sd)
    r = rng.standard_normal(V) * 0.1
    r = np.round(r * 64) / 64  # heavy ties: long runs, tie flags
    rows.append(r)
    x = _bf16(np.stack(rows).astype(np.float32))
    H = 400
    hist = rng.integers(0, V, size=x.shape[0] * H).astype(np.int32)
    offs = (np.arange(x.shape[0] + 1) * H).astype(np.int32)
    for top_p in (0.25, 0.5, float(np.nextafter(np.float32(0.5), np.float32(1))), 0.75, 0.999, 1.0):
        for T, min_p, pen in ((1.3, 0.0, 1.0), (0.6, 0.0, 1.2), (1.0, 0.02, 1.0)):
            w = small_workload(f"skip-p{top_p}-T{T}-m{min_p}-r{pen}", x,
                               dict(temperature=T, top_k=0, top_p=top_p, min_p=min_p, softcap=30.0,
                                    repetition_penalty=pen),
                               history=hist, offsets=offs,
                               uniforms=W.mt_uniforms(int(top_p * 1000) + int(T * 10), x.shape[0]), dtype="bf16")
            _check(sampler, w)
