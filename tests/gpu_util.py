"""Shared helpers for the GPU parity tests: run a workload through the HIP
library (via the C ABI) and through the CPU oracle on identical inputs."""
from __future__ import annotations

import numpy as np

import ge_oracle as O
from gemmaedge_amd import workloads as W


def oracle_params(p: dict) -> O.Params:
    return O.make_params(**p)


to_device = W.to_device


def run_gpu(sampler, w: W.Workload):
    import torch

    from gemmaedge_amd import SamplingConfig

    logits, hist, offs, uni = to_device(w)
    cfg = SamplingConfig(**{k: v for k, v in w.params.items()})
    tokens, probs, flags = sampler.sample(logits, cfg, uniforms=uni, history=hist,
                                          history_offsets=offs)
    torch.cuda.synchronize()
    return tokens.cpu().numpy(), probs.cpu().numpy(), flags.cpu().numpy()


def run_oracle(w: W.Workload, nthreads: int = 0):
    hist = w.history if w.history.size else None
    offs = w.offsets if w.history.size else None
    return O.run(w.logits, oracle_params(w.params), history=hist, offsets=offs,
                 uniforms=w.uniforms, nthreads=nthreads)


def assert_parity(w: W.Workload, gpu, ora, label=""):
    tokens, probs, flags = gpu
    bad = np.nonzero(tokens != ora.tokens)[0]
    assert bad.size == 0, (
        f"{label or w.name}: {bad.size} token mismatches, first rows {bad[:8].tolist()} "
        f"gpu {tokens[bad[:8]].tolist()} oracle {ora.tokens[bad[:8]].tolist()}")
    # Probabilities: bit-identical (same arithmetic); NaN only where the oracle has NaN.
    pb = probs.view(np.uint32)
    ob = ora.probs.view(np.uint32)
    both_nan = np.isnan(probs) & np.isnan(ora.probs)
    pbad = np.nonzero((pb != ob) & ~both_nan)[0]
    assert pbad.size == 0, (
        f"{label or w.name}: prob mismatch rows {pbad[:8].tolist()} gpu {probs[pbad[:8]]} "
        f"oracle {ora.probs[pbad[:8]]}")
    fbad = np.nonzero((flags & 1) != ora.flags)[0]
    assert fbad.size == 0, f"{label or w.name}: near-boundary flag mismatch rows {fbad[:8].tolist()}"


def small_workload(name, logits, params, history=None, offsets=None, uniforms=None, dtype="f32"):
    logits = np.ascontiguousarray(logits)
    if logits.ndim == 1:
        logits = logits[None, :]
    rows = logits.shape[0]
    if history is None:
        history = np.zeros(0, np.int32)
        offsets = np.zeros(rows + 1, np.int32)
    if uniforms is None:
        uniforms = W.mt_uniforms(7, rows)
    full = dict(temperature=1.0, top_k=64, top_p=0.95, min_p=0.0, softcap=0.0,
                repetition_penalty=1.0)
    full.update(params)
    return W.Workload(name, logits, dtype, full, np.asarray(history, np.int32),
                      np.asarray(offsets, np.int32), np.asarray(uniforms, np.float32))
