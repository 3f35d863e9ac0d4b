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


@pytest.mark.parametrize("mode", ["lib", "cli"])
def test_generate_loop_matches_oracle(tmp_path, mode):
    """The decode loop through the drop-in (tests/cpp/drop_in_test.cpp
    generate mode): Gemma4Session::generate (src/generation.cpp:452-469) or the
    CLI loop (src/main.cpp:138-146) over a table of logits rows, one
    mt19937_64 across greedy and sampling steps, prompt + generated ids as the
    penalty history, stop tokens {1, 106}. The oracle replays the same loop;
    the step that lifts token 106 ends it (mode lib keeps the stop token in the
    output, mode cli drops it), as core_tests.cpp:473-504 checks for greedy."""
    rng = np.random.default_rng(41)
    rows, vocab, seed, stop_step = 30, 262144, 1234, 23
    x = (rng.standard_normal((rows, vocab)) * 3).astype(np.float32)
    peaks = rng.choice(np.arange(200, vocab), size=12, replace=False)
    x[:, peaks] += 7.0  # recurring candidates: the penalty history matters
    x[stop_step, 106] = 80.0
    prompt = rng.integers(0, vocab, size=32).astype(np.int32)
    temps = [1.0, 0.0, 0.7, 1.3, 0.0]
    x.tofile(tmp_path / "rows.bin")
    prompt.tofile(tmp_path / "prompt.bin")
    got = _run(["generate", tmp_path / "rows.bin", rows, vocab, seed, tmp_path / "prompt.bin", prompt.size,
                ",".join(str(t) for t in temps), mode])
    eng = W.MT19937_64(seed)
    hist = list(prompt)
    want = []
    for i in range(rows):
        t = temps[i % len(temps)]
        u = W.canonical_float(eng()) if t > 0 else 0.0
        h = np.array(hist, np.int32)
        ora = O.run(x[i:i + 1], O.make_params(temperature=t, top_k=64, top_p=0.95, softcap=30.0,
                                              repetition_penalty=1.1),
                    history=h, offsets=np.array([0, h.size], np.int32),
                    uniforms=np.array([u], np.float32), nthreads=1)
        tok = int(ora.tokens[0])
        stop = tok in (1, 106)
        if mode == "cli" and stop:
            break
        want.append(tok)
        if stop:
            break
        hist.append(tok)
    assert len(want) == stop_step + (1 if mode == "lib" else 0)
    assert got == want


@pytest.mark.parametrize("env", [
    {"GEMMAEDGE_TEMPERATURE": "0.7", "GEMMAEDGE_TOP_K": "40", "GEMMAEDGE_TOP_P": "0.9", "GEMMAEDGE_MIN_P": "0.02",
     "GEMMAEDGE_SEED": "77", "GEMMAEDGE_SOFTCAP": "30", "GEMMAEDGE_REPETITION_PENALTY": "1.15"},
    {"GEMMAEDGE_TEMPERATURE": " 0 ", "GEMMAEDGE_SOFTCAP": "30.0", "GEMMAEDGE_REPETITION_PENALTY": "1.3"},
    {"GEMMAEDGE_TOP_K": "not-a-number", "GEMMAEDGE_SEED": "5", "GEMMAEDGE_TOP_P": "1e-50"},
])
def test_env_config_matches_oracle(tmp_path, env):
    """The configuration surface (include/gemmaedge/sampling_env.h) driving
    GPU samples: drop_in_test env reads every field through
    sampling_config_from_env / sampling_extras_from_env (malformed values keep
    the default, an underflowing decimal gives its finite value); the oracle
    uses the same fields, parsed by SamplingConfig.from_env."""
    from gemmaedge_amd import SamplingConfig

    rng = np.random.default_rng(61)
    rows, vocab, hl = 8, 262144, 64
    x = (rng.standard_normal((rows, vocab)) * 3).astype(np.float32)
    hist = rng.integers(0, vocab, size=(rows, hl)).astype(np.int32)
    x.tofile(tmp_path / "rows.bin")
    hist.tofile(tmp_path / "hist.bin")
    full = dict(os.environ)
    for k in list(full):
        if k.startswith("GEMMAEDGE_"):
            del full[k]
    full.update(env)
    print("[dropin] env", env, flush=True)
    r = subprocess.run([BIN, "env", str(tmp_path / "rows.bin"), str(rows), str(vocab), str(tmp_path / "hist.bin"),
                        str(hl)], capture_output=True, text=True, timeout=120, env=full)
    assert r.returncode == 0, r.stderr
    got = [int(t) for t in r.stdout.split()]
    cfg = SamplingConfig.from_env(SamplingConfig(softcap=0.0, repetition_penalty=1.0), environ=full)
    u = W.mt_uniforms(cfg.seed, rows) if cfg.temperature > 0 else np.zeros(rows, np.float32)
    ora = O.run(x, O.make_params(temperature=cfg.temperature, top_k=cfg.top_k, top_p=cfg.top_p, min_p=cfg.min_p,
                                 softcap=cfg.softcap, repetition_penalty=cfg.repetition_penalty),
                history=hist.reshape(-1), offsets=(np.arange(rows + 1) * hl).astype(np.int32), uniforms=u)
    assert got == ora.tokens.tolist()
