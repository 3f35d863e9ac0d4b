"""GPU parity of the single-pass selection kernel (shared parameters, top-k at
most 64, temperature > 0, penalty >= 1, rows of at most 16 chunks of 16,384
logits with enough rows to fill 16 chunks). Every case is shaped so that the
call plan routes it there, and compared bit for bit with the CPU oracle,
including the rows whose candidate lists do not certify and take the exact
rescans. The list area must be zero between calls whatever the previous
call's shape, so shapes alternate on one handle."""
import numpy as np
import pytest

from gemmaedge_amd import workloads as W
from gpu_util import assert_parity, run_gpu, run_oracle, small_workload

pytestmark = pytest.mark.gpu

CHUNK = 256 * 64


def stream_shape(V):
    """(cpr, rows needed) for a vocabulary the single-pass kernel takes."""
    cpr = -(-V // CHUNK)
    assert cpr <= 16
    return cpr, -(-16 // cpr)


@pytest.fixture(scope="module")
def sampler():
    import torch

    from gemmaedge_amd import Sampler, available

    assert torch.cuda.is_available(), "GPU test run without a GPU"
    assert available(), "no gfx950 device visible to the HIP library"
    s = Sampler(max_rows=64, max_vocab=W.VOCAB, max_history=4096)
    yield s
    s.close()


def _check(sampler, w, label=""):
    print(f"[stream] {label or w.name} rows={w.rows} V={w.vocab} {w.dtype} {w.params}", flush=True)
    gpu = run_gpu(sampler, w)
    ora = run_oracle(w)
    assert_parity(w, gpu, ora, label)
    return gpu, ora


def _logits(rng, kind, rows, V):
    if kind == "normal":
        return (rng.standard_normal((rows, V)) * rng.uniform(0.1, 5)).astype(np.float32)
    if kind == "peaks":
        x = (rng.standard_normal((rows, V)) * 3).astype(np.float32)
        for r in range(rows):
            idx = rng.choice(V, size=int(rng.integers(8, 33)), replace=False)
            x[r, idx] += rng.uniform(6, 10, size=idx.size).astype(np.float32)
        return x
    if kind == "ties":
        return rng.integers(-3, 4, size=(rows, V)).astype(np.float32)
    if kind == "plateau":  # softcap saturation: many capped values tie
        return (rng.standard_normal((rows, V)) * 200).astype(np.float32)
    if kind == "zeros":  # +-0 and tiny values
        return rng.choice(np.array([0.0, -0.0, 1e-30, -1e-30, 2.0], np.float32), size=(rows, V))
    if kind == "desc":  # the whole top-k in the first chunk
        return np.ascontiguousarray(-np.sort(rng.standard_normal((rows, V)).astype(np.float32), axis=1))
    if kind == "asc":
        return np.ascontiguousarray(np.sort(rng.standard_normal((rows, V)).astype(np.float32), axis=1))
    if kind == "hot":  # one hot region inside one wave's slots
        x = rng.standard_normal((rows, V)).astype(np.float32)
        a = int(rng.integers(0, max(V - 300, 1)))
        x[:, a:a + 300] += 6.0
        return x
    if kind == "nan":
        x = (rng.standard_normal((rows, V)) * 3).astype(np.float32)
        x[rng.random((rows, V)) < 0.01] = np.nan
        return x
    if kind == "nanwave":  # whole waves of NaN: waves without a bound
        x = (rng.standard_normal((rows, V)) * 3).astype(np.float32)
        x[:, : min(V, 8192)] = np.nan
        return x
    if kind == "masked":  # a few finite logits, the rest -inf
        x = np.full((rows, V), -np.inf, np.float32)
        for r in range(rows):
            x[r, rng.choice(V, 10, replace=False)] = rng.standard_normal(10).astype(np.float32) * 3
        return x
    if kind == "maskedwide":  # more finite logits than k, the rest -inf (constrained decoding)
        x = np.full((rows, V), -np.inf, np.float32)
        for r in range(rows):
            x[r, rng.choice(V, 300, replace=False)] = rng.standard_normal(300).astype(np.float32) * 3
        return x
    if kind == "halfmasked":  # -inf over a contiguous half of the row
        x = (rng.standard_normal((rows, V)) * 3).astype(np.float32)
        x[:, V // 4: V // 4 + V // 2] = -np.inf
        return x
    raise ValueError(kind)


KINDS = ["normal", "peaks", "ties", "plateau", "zeros", "desc", "asc", "hot", "nan", "nanwave", "masked",
         "maskedwide", "halfmasked"]
VOCABS = [262144, 262143, 200001, 152064, 100003, 40000, 16384, 16385]


def _case(rng, case, kind=None, V=None, dtype="f32"):
    V = int(rng.choice(VOCABS)) if V is None else V
    _, need = stream_shape(V)
    rows = need + int(rng.integers(0, 3))
    kind = kind or str(rng.choice(KINDS))
    x = _logits(rng, kind, rows, V)
    params = dict(temperature=float(rng.choice([0.5, 0.7, 1.0, 1.7])),
                  top_k=int(rng.choice([1, 2, 5, 17, 40, 64])),
                  top_p=float(rng.choice([0.0, 0.5, 0.9, 0.95, 1.0])),
                  min_p=float(rng.choice([0.0, 0.0, 0.05, 0.5])),
                  softcap=float(rng.choice([0.0, 30.0, 5.0])),
                  repetition_penalty=float(rng.choice([1.0, 1.1, 1.5, np.inf])))
    H = int(rng.choice([0, 7, 300, 2048]))
    hist = rng.integers(-2, V + 2, size=rows * H).astype(np.int32)  # includes out-of-range ids
    offsets = (np.arange(rows + 1) * H).astype(np.int32)
    if dtype == "bf16":
        x = W.f32_to_bf16_bits(np.nan_to_num(x, nan=0.0, posinf=3e38, neginf=-3e38))
    return small_workload(f"stream{case}-{kind}-V{V}", x, params, hist, offsets, W.mt_uniforms(1000 + case, rows),
                          dtype=dtype)


def test_stream_random_cases(sampler):
    rng = np.random.default_rng(31337)
    for case in range(48):
        _check(sampler, _case(rng, case))


@pytest.mark.parametrize("kind", KINDS)
def test_stream_each_distribution(sampler, kind):
    rng = np.random.default_rng(100 + KINDS.index(kind))
    for i, V in enumerate((262144, 152064)):
        _check(sampler, _case(rng, 500 + i, kind=kind, V=V))


def test_stream_bf16(sampler):
    rng = np.random.default_rng(77)
    for case in range(12):
        _check(sampler, _case(rng, 700 + case, dtype="bf16"))


def test_stream_benchmark_rows(sampler):
    # C2 at full size and C1 (one row: 16 chunks), as the benchmark runs them.
    _check(sampler, W.c2())
    _check(sampler, W.c1())
    for seed in range(2, 6):
        _check(sampler, W.c1(seed=seed))


def test_stream_alternating_shapes(sampler):
    # Calls of different shapes on one handle: the list words each call reads
    # must all have been cleared by the previous calls' merges, whatever
    # their layout (lists per row and words per list differ with the vocab).
    rng = np.random.default_rng(4096)
    seq = [262144, 16384, 152064, 262144, 40000, 100003, 262144, 16385, 200001, 262144]
    for i, V in enumerate(seq):
        _check(sampler, _case(rng, 900 + i, kind="peaks", V=V))


def test_stream_mixed_shapes_in_one_graph(sampler):
    # Launches of different shapes on one handle captured back to back in one
    # graph (no host wait between kernels), the graph replayed three times:
    # every call's list area must be zero when it starts, whichever call of
    # which shape ran before it, and every replay must give the same outputs.
    import ctypes

    import torch

    from gemmaedge_amd import sampler as S

    rng = np.random.default_rng(555)
    seq = [262144, 16384, 152064, 262144, 40000, 262144, 100003, 16385]
    cases = [_case(rng, 1200 + i, kind=str(rng.choice(["normal", "peaks", "ties"])), V=V) for i, V in enumerate(seq)]
    dev = []
    for w in cases:
        logits, hist, offs, uni = W.to_device(w)
        outs = (torch.empty(w.rows, dtype=torch.int32, device="cuda"),
                torch.empty(w.rows, dtype=torch.float32, device="cuda"),
                torch.empty(w.rows, dtype=torch.int32, device="cuda"))
        a = S.SampleArgs()
        a.logits, a.dtype, a.rows, a.vocab, a.row_stride = logits.data_ptr(), S.GE_DTYPE_F32, w.rows, w.vocab, w.vocab
        a.params = S.SamplingConfig(**w.params).params()
        if hist is not None:
            a.history, a.history_offsets = hist.data_ptr(), offs.data_ptr()
        a.uniforms = uni.data_ptr()
        a.tokens_out, a.probs_out, a.flags_out = (t.data_ptr() for t in outs)
        dev.append((w, (logits, hist, offs, uni), outs, a))
    lib = S.load_library()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            cs = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            for _, _, _, a in dev:
                assert lib.ge_sample(sampler._h, cs, ctypes.byref(a)) == 0, S.last_error()
    torch.cuda.synchronize()
    oras = [run_oracle(w) for w, _, _, _ in dev]
    for rep in range(3):
        for _, _, outs, _ in dev:
            outs[0].fill_(-7)
        g.replay()
        _ = sum(float(x[0].float().sum()) for _, x, _, _ in dev)  # eager work between replays
        torch.cuda.synchronize()
        for (w, _, outs, _), ora in zip(dev, oras):
            gpu = tuple(x.cpu().numpy() for x in outs)
            assert_parity(w, gpu, ora, f"{w.name} replay {rep}")
