"""A seeded random sweep over every sampling path against the CPU oracle:
vocabularies from 1,000 to 262,144 (aligned and not, one chunk and many), f32
and bf16, narrow, wide, tied, peaked, integer, huge and -inf-masked rows,
greedy to hot temperatures, top-k from 1 to above the selection limit and
off, top-p and min-p cuts, softcaps, penalties above and below 1 with
histories of up to 3,000 ids (with duplicates and out-of-range ids). Tokens
and probabilities must be bit-identical and the near-boundary flags agree."""
import numpy as np
import pytest

from gemmaedge_amd import workloads as W
from gpu_util import assert_parity, run_gpu, run_oracle, small_workload

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sampler():
    import torch

    from gemmaedge_amd import Sampler, available

    assert torch.cuda.is_available(), "GPU test run without a GPU"
    assert available(), "no gfx950 device visible to the HIP library"
    s = Sampler(max_rows=64, max_vocab=W.VOCAB, max_history=20000)
    yield s
    s.close()


def _case(rng, case):
    V = int(rng.choice([1000, 1025, 4099, 16384, 16385, 40000, 70001, 100003, 262144]))
    rows = int(rng.integers(1, 13))
    dtype = str(rng.choice(["f32", "bf16"]))
    kind = int(rng.integers(0, 6))
    if kind == 0:
        x = rng.standard_normal((rows, V)) * rng.uniform(0.03, 5)
    elif kind == 1:
        x = np.round(rng.standard_normal((rows, V)) * rng.uniform(0.05, 1) * 32) / 32
    elif kind == 2:
        x = rng.standard_normal((rows, V)) * 0.1
        x[:, rng.integers(0, V, 8)] += 6
    elif kind == 3:
        x = rng.integers(-3, 4, size=(rows, V)).astype(np.float64)
    elif kind == 4:
        x = rng.standard_normal((rows, V)) * 200
    else:
        x = rng.standard_normal((rows, V)) * 0.5
        x[rng.random((rows, V)) < rng.uniform(0.0, 0.99)] = -np.inf
    x = x.astype(np.float32)
    if dtype == "bf16":
        x = W.f32_to_bf16_bits(x)
    params = dict(temperature=float(rng.choice([0.0, 0.3, 0.7, 1.0, 1.3, 2.0])),
                  top_k=int(rng.choice([0, 0, 1, 8, 40, 64, 100, 1024, 1025, 5000])),
                  top_p=float(rng.choice([0.1, 0.5, 0.9, 0.95, 0.999, 1.0, 1.5])),
                  min_p=float(rng.choice([0.0, 0.0, 0.05, 0.3])),
                  softcap=float(rng.choice([0.0, 30.0, 5.0])),
                  repetition_penalty=float(rng.choice([1.0, 1.0, 1.1, 1.5, 0.8])))
    H = int(rng.choice([0, 1, 64, 500, 3000]))
    hist = rng.integers(-2, V + 2, size=rows * H).astype(np.int32)
    offs = (np.arange(rows + 1) * H).astype(np.int32)
    name = f"sweep{case}: V={V} rows={rows} {dtype} kind={kind} H={H} {params}"
    return small_workload(name, x, params, hist, offs, W.mt_uniforms(9000 + case, rows), dtype=dtype)


@pytest.mark.parametrize("block", range(4))
def test_random_sweep(sampler, block):
    rng = np.random.default_rng(1000 + block)
    for case in range(block * 250, block * 250 + 250):
        w = _case(rng, case)
        print(w.name, flush=True)
        assert_parity(w, run_gpu(sampler, w), run_oracle(w), w.name)
