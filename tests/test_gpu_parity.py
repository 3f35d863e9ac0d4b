"""GPU parity: the HIP sampling path (through the C ABI) against the CPU oracle
on identical logits, histories and uniforms. Token ids and probabilities must
be bit-identical; near-boundary flags must agree."""
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
    s = Sampler(max_rows=512, max_vocab=W.VOCAB, max_history=8192)
    yield s
    s.close()


def _check(sampler, w, label=""):
    print(f"[parity] {label or w.name} rows={w.rows} V={w.vocab} {w.dtype} {w.params}", flush=True)
    gpu = run_gpu(sampler, w)
    ora = run_oracle(w)
    assert_parity(w, gpu, ora, label)
    return gpu, ora


def test_reference_known_answers(sampler):
    # tests/core_tests.cpp:303 — greedy on {-1, 3, 2} selects 1.
    w = small_workload("kat-greedy", np.array([-1.0, 3.0, 2.0], np.float32), dict(temperature=0.0))
    gpu, _ = _check(sampler, w)
    assert gpu[0][0] == 1
    # tests/core_tests.cpp:310 — top_k=1, top_p=1, T=1 on {4, 1, 0} selects 0.
    w = small_workload("kat-topk1", np.array([4.0, 1.0, 0.0], np.float32),
                       dict(temperature=1.0, top_k=1, top_p=1.0))
    gpu, _ = _check(sampler, w)
    assert gpu[0][0] == 0
    # tests/core_tests.cpp:496-500 relies on first-maximum greedy ties.
    w = small_workload("kat-greedy-ties", np.ones(5, np.float32), dict(temperature=0.0))
    gpu, _ = _check(sampler, w)
    assert gpu[0][0] == 0


def test_c1(sampler):
    _check(sampler, W.c1())


def test_c1_greedy(sampler):
    _check(sampler, W.c1(greedy=True))


def test_c2(sampler):
    _check(sampler, W.c2())


def test_c3_rows(sampler):
    _check(sampler, W.c3(rows=24))


def test_c2_bf16(sampler):
    w = W.c2(rows=16)
    w.logits = W.f32_to_bf16_bits(w.logits)
    w.dtype = "bf16"
    _check(sampler, w, "C2-bf16")


def test_c5_steps_with_history(sampler):
    # Each step's history = previously sampled tokens (explicit history form).
    w = W.c5_steps(steps=6)
    toks = []
    for s in range(w.rows):
        hist = np.array(toks, np.int32)
        ws = small_workload(f"C5-step{s}", w.logits[s], w.params, history=hist,
                            offsets=np.array([0, hist.size], np.int32), uniforms=w.uniforms[s:s + 1])
        gpu, ora = _check(sampler, ws)
        toks.append(int(gpu[0][0]))


def _random_case(rng, case):
    V = int(rng.choice([1, 2, 3, 5, 17, 64, 100, 1000, 4096, 4099, 20000, 70001]))
    rows = int(rng.integers(1, 5))
    kind = rng.integers(0, 4)
    if kind == 0:
        x = rng.standard_normal((rows, V)).astype(np.float32) * np.float32(rng.uniform(0.1, 5))
    elif kind == 1:  # heavy ties
        x = rng.integers(-3, 4, size=(rows, V)).astype(np.float32)
    elif kind == 2:  # softcap saturation plateau
        x = (rng.standard_normal((rows, V)) * 200).astype(np.float32)
    else:  # ties at +-0 and small values
        x = rng.choice(np.array([0.0, -0.0, 1e-30, -1e-30, 2.0], np.float32), size=(rows, V))
    temperature = float(rng.choice([0.0, 0.5, 1.0, 1.7]))
    top_k = int(rng.choice([1, 2, 5, 40, 64, 300, 1024]))
    params = dict(temperature=temperature, top_k=top_k,
                  top_p=float(rng.choice([0.0, 0.5, 0.9, 0.95, 1.0, 1.5])),
                  min_p=float(rng.choice([0.0, 0.0, 0.05, 0.5])),
                  softcap=float(rng.choice([0.0, 30.0, 5.0])),
                  repetition_penalty=float(rng.choice([1.0, 1.1, 1.5, 0.8])))
    H = int(rng.choice([0, 1, 7, 64, 300]))
    hist = rng.integers(-2, V + 2, size=rows * H).astype(np.int32)  # includes out-of-range ids
    offsets = (np.arange(rows + 1) * H).astype(np.int32)
    uniforms = W.mt_uniforms(case, rows)
    return small_workload(f"rand{case}", x, params, hist, offsets, uniforms)


def test_random_small_cases(sampler):
    rng = np.random.default_rng(1234)
    for case in range(120):
        _check(sampler, _random_case(rng, case))


def test_nan_logits(sampler):
    x = np.array([np.nan, 1.0, 3.0, np.nan, 3.0, -np.inf, np.inf], np.float32)
    for T in (0.0, 1.0):
        w = small_workload("nan", x, dict(temperature=T, top_k=3, softcap=30.0))
        _check(sampler, w)
    # std::max_element keeps index 0 when it holds NaN.
    w = small_workload("nan0-greedy", np.array([np.nan, 5.0, 1.0], np.float32), dict(temperature=0.0))
    gpu, _ = _check(sampler, w)
    assert gpu[0][0] == 0


def test_unaligned_rows(sampler):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 4099)).astype(np.float32)
    w = small_workload("unaligned", x, dict(temperature=0.8, top_k=50, softcap=30.0))
    _check(sampler, w)
    wb = small_workload("unaligned-bf16", W.f32_to_bf16_bits(x), dict(temperature=0.8, top_k=50),
                        dtype="bf16")
    _check(sampler, wb)


def test_per_row_params(sampler):
    import torch

    from gemmaedge_amd import SamplingConfig

    rng = np.random.default_rng(9)
    rows, V = 6, 50000
    x = (rng.standard_normal((rows, V)) * 3).astype(np.float32)
    cfgs = [SamplingConfig(temperature=t, top_k=k, top_p=p, softcap=30.0, repetition_penalty=1.1)
            for t, k, p in [(0.0, 64, 0.9), (1.0, 64, 0.95), (0.7, 40, 0.9), (1.0, 1024, 0.99),
                            (1.2, 5, 1.0), (0.5, 1, 0.5)]]
    hist = rng.integers(0, V, size=rows * 32).astype(np.int32)
    offs = (np.arange(rows + 1) * 32).astype(np.int32)
    uni = W.mt_uniforms(11, rows)
    tokens, probs, flags = sampler.sample(
        torch.from_numpy(x).cuda(), cfgs, uniforms=torch.from_numpy(uni).cuda(),
        history=torch.from_numpy(hist).cuda(), history_offsets=torch.from_numpy(offs).cuda())
    torch.cuda.synchronize()
    params = [O.make_params(temperature=c.temperature, top_k=c.top_k, top_p=c.top_p,
                            softcap=c.softcap, repetition_penalty=c.repetition_penalty) for c in cfgs]
    ora = O.run(x, params, history=hist, offsets=offs, uniforms=uni)
    assert np.array_equal(tokens.cpu().numpy(), ora.tokens)
    assert np.array_equal(probs.cpu().numpy().view(np.uint32), ora.probs.view(np.uint32))


def test_massive_ties_are_exact(sampler):
    # All-equal logits: every chunk's candidates overflow LDS, so the exact
    # routine (radix select, lowest indices of the tie class) runs, and the
    # merge must rescan the low chunks: the top-k are indices 0..k-1.
    for k in (1, 64, 1024):
        w = small_workload(f"all-equal-k{k}", np.zeros(200000, np.float32), dict(temperature=1.0, top_k=k))
        _check(sampler, w)
    # Masked vocabulary: a few finite logits, the rest -inf (softcap maps
    # them to -30, a tie class of ~262k tokens that top-k 64 reaches).
    rng = np.random.default_rng(21)
    x = np.full((2, W.VOCAB), -np.inf, np.float32)
    for r in range(2):
        x[r, rng.choice(W.VOCAB, 10, replace=False)] = rng.standard_normal(10).astype(np.float32) * 3
    _check(sampler, small_workload("masked", x, dict(temperature=1.0, top_k=64, softcap=30.0)))
    _check(sampler, small_workload("masked-nocap", x, dict(temperature=0.7, top_k=40, top_p=1.0)))
    # Ties with a penalty on part of the tie class.
    hist = np.arange(0, 5000, 3, dtype=np.int32)
    w = small_workload("ties-penalty", np.ones(100000, np.float32), dict(temperature=1.0, top_k=300,
                       repetition_penalty=1.3), history=hist, offsets=np.array([0, hist.size], np.int32))
    _check(sampler, w)


@pytest.mark.parametrize("rows", [1, 64])
def test_clustered_top_k_takes_the_rescan(sampler, rows):
    # Each chunk lists only about k / chunks + 5 sigma entries; when the row's
    # top-k sits in one chunk (sorted logits, or one hot region) the merge
    # rescans that chunk with m = k. Results must still be exact.
    rng = np.random.default_rng(33 + rows)
    V = W.VOCAB
    base = rng.standard_normal((rows, V)).astype(np.float32)
    desc = -np.sort(base, axis=1)                     # descending: top-k in chunk 0
    asc = np.sort(base, axis=1)                       # ascending: top-k in the last chunk
    hot = base.copy()
    hot[:, 70000:72000] += 6.0                        # one hot region
    for name, x in (("desc", desc), ("asc", asc), ("hot", hot)):
        for k, T, p in ((40, 0.7, 0.9), (64, 1.0, 0.95), (1024, 1.0, 0.99)):
            hist = rng.integers(0, V, size=rows * 64).astype(np.int32)
            offs = (np.arange(rows + 1) * 64).astype(np.int32)
            w = small_workload(f"{name}-k{k}-r{rows}", np.ascontiguousarray(x),
                               dict(temperature=T, top_k=k, top_p=p, softcap=30.0, repetition_penalty=1.15),
                               history=hist, offsets=offs, uniforms=W.mt_uniforms(k + rows, rows))
            _check(sampler, w)


def test_repeated_rescans_are_stable(sampler):
    # Regression: every row of sorted logits takes the merge's rescan
    # fallback; repeated launches on one handle, with no host wait between
    # the kernels of consecutive launches, must all match (a scratch
    # word shared between two LDS helpers once let waves disagree on the
    # fallback decision in about 1% of launches).
    import torch

    from gemmaedge_amd import SamplingConfig

    rows, V = 64, W.VOCAB
    rng = np.random.default_rng(97)
    x = np.ascontiguousarray(-np.sort(rng.standard_normal((rows, V)).astype(np.float32), axis=1))
    hist = rng.integers(0, V, size=rows * 64).astype(np.int32)
    offs = (np.arange(rows + 1) * 64).astype(np.int32)
    dx, dh, do = (torch.from_numpy(a).cuda() for a in (x, hist, offs))
    for k, T, p in ((40, 0.7, 0.9), (64, 1.0, 0.95)):
        uni = W.mt_uniforms(k, rows)
        ora = O.run(x, O.make_params(temperature=T, top_k=k, top_p=p, softcap=30.0, repetition_penalty=1.15),
                    history=hist, offsets=offs, uniforms=uni)
        cfg = SamplingConfig(temperature=T, top_k=k, top_p=p, softcap=30.0, repetition_penalty=1.15)
        du = torch.from_numpy(uni).cuda()
        # Shared parameters take the single-pass kernel (polled lists); the
        # same parameters per row take select_kernel (lists and tickets).
        for label, c in (("shared", cfg), ("per-row", [cfg] * rows)):
            bad = 0
            for _ in range(40):
                t, _, _ = sampler.sample(dx, c, uniforms=du, history=dh, history_offsets=do)
                bad += int(np.count_nonzero(t.cpu().numpy() != ora.tokens))
            assert bad == 0, f"k={k} {label}: {bad} mismatching row-launches over 40 launches"


def test_penalty_below_one_with_long_histories(sampler):
    # r < 1 raises penalised positive logits, so every penalised token of a
    # chunk is listed besides its top m. About 250 history ids per chunk
    # overflow a chunk's slot: it publishes a failed guarantee and the merge
    # rescans it exactly. About 40 per chunk fit, and the appended entries
    # take part in the merge.
    rng = np.random.default_rng(55)
    rows, V = 8, W.VOCAB
    x = (rng.standard_normal((rows, V)) * 3).astype(np.float32)
    for H in (640, 4096):
        hist = rng.integers(0, V, size=rows * H).astype(np.int32)
        offs = (np.arange(rows + 1) * H).astype(np.int32)
        w = small_workload(f"pen0.8-H{H}", x, dict(temperature=0.7, top_k=40, top_p=0.9, softcap=30.0,
                                                     repetition_penalty=0.8),
                           history=hist, offsets=offs, uniforms=W.mt_uniforms(H, rows))
        _check(sampler, w)


@pytest.mark.parametrize("k", [40, 1024])
def test_penalty_below_one_dense_history(sampler, k):
    # r < 1 with thousands of unique history ids inside one chunk: more
    # penalised tokens than the exact chunk routine can stage. It keeps the
    # chunk's top k penalised tokens by final value besides its top k
    # unpenalised ones, so no row is refused (no GE_FLAG_UNSUPPORTED).
    from gemmaedge_amd import sampler as S

    rng = np.random.default_rng(1000 + k)
    rows, V = 4, W.VOCAB
    x = (rng.standard_normal((rows, V)) * 3).astype(np.float32)
    H = 6000
    hist = np.concatenate([
        np.concatenate([16384 * (r + 1) + 500 + np.arange(5000), rng.integers(0, V, size=H - 5000)])
        for r in range(rows)]).astype(np.int32)
    offs = (np.arange(rows + 1) * H).astype(np.int32)
    w = small_workload(f"pen0.8-dense-k{k}", x, dict(temperature=1.0 if k > 64 else 0.7, top_k=k,
                                                      top_p=0.99 if k > 64 else 0.9, softcap=30.0,
                                                      repetition_penalty=0.8),
                       history=hist, offsets=offs, uniforms=W.mt_uniforms(k + 7, rows))
    gpu, _ = _check(sampler, w)
    assert not np.any(gpu[2] & S.GE_FLAG_UNSUPPORTED), gpu[2]


def test_rescan_with_penalised_top_tokens(sampler):
    # Sorted rows put the whole top k in the first chunk, so the merge
    # rescans it with m = k; the history holds its 3000 largest tokens
    # (r > 1 lowers them). The rescan keeps the top k penalised tokens by
    # final value besides the top k unpenalised ones instead of every
    # penalised token above the bound, so it fits and matches the oracle.
    from gemmaedge_amd import sampler as S

    rng = np.random.default_rng(4242)
    rows, V = 2, W.VOCAB
    x = np.ascontiguousarray(-np.sort((rng.standard_normal((rows, V)) * 3).astype(np.float32), axis=1))
    H = 3000
    hist = np.concatenate([np.arange(H), rng.integers(0, V, size=H)]).astype(np.int32)
    offs = np.array([0, H, 2 * H], np.int32)
    for k, r in ((1024, 1.2), (40, 1.5), (256, 0.9)):
        w = small_workload(f"rescan-pen-k{k}-r{r}", x, dict(temperature=1.0, top_k=k, top_p=0.99, softcap=30.0,
                                                             repetition_penalty=r),
                           history=hist, offsets=offs, uniforms=W.mt_uniforms(k, rows))
        gpu, _ = _check(sampler, w)
        assert not np.any(gpu[2] & S.GE_FLAG_UNSUPPORTED), gpu[2]
