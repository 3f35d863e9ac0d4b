"""TEST INFRASTRUCTURE ONLY — ctypes wrapper for the CPU oracle (oracle/lib/libge_oracle.so).

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as
the checker; the product package (gemmaedge_amd) never imports this module.

The oracle restates the reference sampler (src/generation.cpp:60-127) and the
final-logit softcap (src/generation.cpp:431-437); see oracle/ge_oracle.h.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libge_oracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libge_ref.so")

F32 = 0
BF16 = 1


class Params(ctypes.Structure):
    """Same layout as ge_sample_params (include/gemmaedge_sampler.h)."""

    _fields_ = [
        ("temperature", ctypes.c_float),
        ("top_k", ctypes.c_uint32),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("softcap", ctypes.c_float),
        ("repetition_penalty", ctypes.c_float),
    ]


class Result(ctypes.Structure):
    _fields_ = [
        ("token", ctypes.c_int32),
        ("prob", ctypes.c_float),
        ("k", ctypes.c_uint32),
        ("keep", ctypes.c_uint32),
        ("mass", ctypes.c_float),
        ("draw", ctypes.c_float),
        ("denominator", ctypes.c_double),
        ("position", ctypes.c_uint32),
        ("near_boundary", ctypes.c_int32),
    ]


RESULT_DTYPE = np.dtype(
    [
        ("token", np.int32),
        ("prob", np.float32),
        ("k", np.uint32),
        ("keep", np.uint32),
        ("mass", np.float32),
        ("draw", np.float32),
        ("denominator", np.float64),
        ("position", np.uint32),
        ("near_boundary", np.int32),
    ],
    align=True,
)
assert RESULT_DTYPE.itemsize == ctypes.sizeof(Result)


def make_params(temperature=1.0, top_k=64, top_p=0.95, min_p=0.0, softcap=0.0,
                repetition_penalty=1.0) -> Params:
    """Defaults are the reference SamplingConfig (include/gemmaedge/generation.h:55-61)
    with no softcap and no penalty."""
    return Params(temperature, top_k, top_p, min_p, softcap, repetition_penalty)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        L.ge_oracle_uniform_from_u64.restype = ctypes.c_float
        L.ge_oracle_uniform_from_u64.argtypes = [ctypes.c_uint64]
        L.ge_oracle_mt_uniforms.argtypes = [ctypes.c_uint64, sz, vp]
        L.ge_oracle_mt_outputs.argtypes = [ctypes.c_uint64, sz, vp]
        L.ge_oracle_tanhf.restype = ctypes.c_float
        L.ge_oracle_tanhf.argtypes = [ctypes.c_float]
        L.ge_oracle_expf.restype = ctypes.c_float
        L.ge_oracle_expf.argtypes = [ctypes.c_float]
        L.ge_oracle_tanhf_bits.argtypes = [ctypes.c_uint32, sz, vp]
        L.ge_oracle_expf_bits.argtypes = [ctypes.c_uint32, sz, vp]
        L.ge_oracle_transform_row.argtypes = [vp, ctypes.c_int, sz, vp, sz, ctypes.POINTER(Params), vp]
        L.ge_oracle_sample_final.restype = ctypes.c_int
        L.ge_oracle_sample_final.argtypes = [vp, sz, ctypes.POINTER(Params), ctypes.c_float,
                                             ctypes.POINTER(Result)]
        L.ge_oracle_run.restype = ctypes.c_int
        L.ge_oracle_run.argtypes = [vp, ctypes.c_int, ctypes.c_int, sz, sz, vp, ctypes.c_int,
                                    vp, vp, vp, vp, vp, vp, vp, ctypes.c_int]
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def uniform_from_u64(x: int) -> float:
    return float(lib().ge_oracle_uniform_from_u64(x))


def mt_uniforms(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().ge_oracle_mt_uniforms(seed, n, _ptr(out))
    return out


def mt_outputs(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint64)
    lib().ge_oracle_mt_outputs(seed, n, _ptr(out))
    return out


def tanhf_bits(lo: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    lib().ge_oracle_tanhf_bits(lo, n, _ptr(out))
    return out


def expf_bits(lo: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    lib().ge_oracle_expf_bits(lo, n, _ptr(out))
    return out


def transform_row(logits: np.ndarray, params: Params, history=None) -> np.ndarray:
    dtype = BF16 if logits.dtype == np.uint16 else F32
    logits = np.ascontiguousarray(logits)
    out = np.empty(logits.shape[-1], np.float32)
    h = None if history is None else np.ascontiguousarray(history, np.int32)
    lib().ge_oracle_transform_row(_ptr(logits), dtype, logits.shape[-1], _ptr(h),
                                  0 if h is None else h.size, ctypes.byref(params), _ptr(out))
    return out


def sample_final(values: np.ndarray, params: Params, u: float) -> Result:
    values = np.ascontiguousarray(values, np.float32)
    r = Result()
    rc = lib().ge_oracle_sample_final(_ptr(values), values.size, ctypes.byref(params), u,
                                      ctypes.byref(r))
    if rc != 0:
        raise ValueError("cannot sample empty logits")
    return r


@dataclass
class BatchOut:
    tokens: np.ndarray
    probs: np.ndarray
    flags: np.ndarray
    results: np.ndarray


def run(logits: np.ndarray, params, history=None, offsets=None, uniforms=None,
        nthreads: int = 0) -> BatchOut:
    """Full pipeline over a [rows, vocab] batch. `logits` is float32 or uint16 (bf16 bits).
    `params` is one Params or a list of per-row Params."""
    logits = np.ascontiguousarray(logits)
    rows, vocab = logits.shape
    dtype = BF16 if logits.dtype == np.uint16 else F32
    if isinstance(params, Params):
        parr = (Params * 1)(params)
        per_row = 0
    else:
        parr = (Params * rows)(*params)
        per_row = 1
    h = None if history is None else np.ascontiguousarray(history, np.int32)
    o = None if offsets is None else np.ascontiguousarray(offsets, np.int32)
    u = None if uniforms is None else np.ascontiguousarray(uniforms, np.float32)
    tokens = np.empty(rows, np.int32)
    probs = np.empty(rows, np.float32)
    flags = np.empty(rows, np.int32)
    results = np.zeros(rows, RESULT_DTYPE)
    rc = lib().ge_oracle_run(_ptr(logits), dtype, rows, vocab, vocab, ctypes.cast(parr, ctypes.c_void_p),
                             per_row, _ptr(h), _ptr(o), _ptr(u), _ptr(tokens), _ptr(probs),
                             _ptr(flags), _ptr(results), nthreads)
    if rc != 0:
        raise ValueError("oracle rejected arguments")
    return BatchOut(tokens, probs, flags, results)


_ref = None


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref_lib():
    """The reference's own sample_token (oracle/_ref, built from /root/reference)."""
    global _ref
    if _ref is None:
        L = ctypes.CDLL(REF_PATH, mode=os.RTLD_LAZY)
        L.ref_sample_sequence.restype = ctypes.c_int
        L.ref_sample_sequence.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t,
                                          ctypes.c_float, ctypes.c_uint32, ctypes.c_float,
                                          ctypes.c_float, ctypes.c_uint64, ctypes.c_void_p]
        _ref = L
    return _ref


def ref_sample_sequence(logits: np.ndarray, temperature: float, top_k: int, top_p: float,
                        min_p: float, seed: int) -> np.ndarray:
    logits = np.ascontiguousarray(logits, np.float32)
    rows, vocab = logits.shape
    out = np.empty(rows, np.int32)
    rc = ref_lib().ref_sample_sequence(_ptr(logits), rows, vocab, temperature, top_k, top_p,
                                       min_p, seed, _ptr(out))
    if rc != 0:
        raise RuntimeError("reference sample_token raised")
    return out
