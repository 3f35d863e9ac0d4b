"""gemmaedge::sample_token with the reference's signature (C++ drop-in,
include/gemmaedge/sampling.h) on the GPU: the reference's own test_sampling
known answers (tests/core_tests.cpp:298-312), and a seeded stream of rows
sampled with one std::mt19937_64 as Gemma4Session::generate does
(src/generation.cpp:456-460), compared token by token with the oracle."""
import os
import subprocess

import numpy as np
import pytest

import ge_oracle as O
from gemmaedge_amd import workloads as W

pytestmark = pytest.mark.gpu
BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "bin", "drop_in_test")


def _run(args):
    print("[dropin]", " ".join(str(a) for a in args), flush=True)
    r = subprocess.run([BIN] + [str(a) for a in args], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return [int(x) for x in r.stdout.split()]


def test_reference_known_answers():
    assert os.path.exists(BIN), "build tests/cpp first"
    _run([])


@pytest.mark.parametrize("cfg", [(1.0, 64, 0.95, 0.0), (0.7, 40, 0.9, 0.05), (0.0, 64, 0.9, 0.0),
                                 (1.3, 1024, 0.99, 0.0)])
def test_seeded_stream_matches_oracle(tmp_path, cfg):
    rng = np.random.default_rng(17)
    rows, vocab, seed = 12, 262144, 99
    x = (rng.standard_normal((rows, vocab)) * 3).astype(np.float32)
    path = tmp_path / "rows.bin"
    x.tofile(path)
    got = _run([path, rows, vocab, *cfg, seed])
    # one engine output per non-greedy token, in order
    u = W.mt_uniforms(seed, rows) if cfg[0] > 0 else np.zeros(rows, np.float32)
    ora = O.run(x, O.make_params(temperature=cfg[0], top_k=cfg[1], top_p=cfg[2], min_p=cfg[3]),
                uniforms=u)
    assert got == ora.tokens.tolist()


def test_history_overload_matches_oracle(tmp_path):
    rng = np.random.default_rng(23)
    rows, vocab, seed, hl = 6, 50000, 5, 300
    x = (rng.standard_normal((rows, vocab)) * 3).astype(np.float32)
    hist = rng.integers(0, vocab, size=(rows, hl)).astype(np.int32)
    x.tofile(tmp_path / "rows.bin")
    hist.tofile(tmp_path / "hist.bin")
    got = _run([tmp_path / "rows.bin", rows, vocab, 1.0, 64, 0.95, 0.0, seed, 30.0, 1.1,
                tmp_path / "hist.bin", hl])
    u = W.mt_uniforms(seed, rows)
    ora = O.run(x, O.make_params(temperature=1.0, top_k=64, top_p=0.95, softcap=30.0,
                                 repetition_penalty=1.1),
                history=hist.reshape(-1), offsets=(np.arange(rows + 1) * hl).astype(np.int32), uniforms=u)
    assert got == ora.tokens.tolist()
