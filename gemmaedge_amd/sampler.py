"""Python binding of the gfx950 sampling library (include/gemmaedge_sampler.h).

ctypes over lib/libgemmaedge_sampler.so; torch supplies device memory and
streams. The binding fails loudly when the library or a gfx950 device is
missing: there is no CPU fallback on this path.

Mirrors the reference interface: ``SamplingConfig`` has the fields and defaults
of include/gemmaedge/generation.h:55-61 and ``sample_token`` the behaviour of
src/generation.cpp:60-127 (empty logits raise ValueError, the counterpart of
std::invalid_argument at :63).
"""
from __future__ import annotations

import ctypes
import dataclasses
import math
import os
import re
import struct
from dataclasses import dataclass
from typing import Optional, Sequence

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libgemmaedge_sampler.so")

GE_OK = 0
GE_ERR_INVALID_ARG = -1
GE_ERR_UNSUPPORTED = -2
GE_ERR_DEVICE = -3
GE_ERR_NO_DEVICE = -4
GE_ERR_CAPACITY = -5

GE_DTYPE_F32 = 0
GE_DTYPE_BF16 = 1

GE_FLAG_NEAR_BOUNDARY = 1
GE_FLAG_UNSUPPORTED = 2
GE_FLAG_STOP = 4
GE_FLAG_DONE = 8
GE_FLAG_TIMEOUT = 16

GE_STOP_AFTER_PUSH = 0   # Gemma4Session::generate (src/generation.cpp:461-465)
GE_STOP_BEFORE_PUSH = 1  # CLI decode loop (src/main.cpp:140-143)
GE_MAX_STOP_TOKENS = 64
GE_NOALLOC_MAX_ROWS = 512

EXPORTS = (
    "ge_sampler_available",
    "ge_sampler_create",
    "ge_sampler_destroy",
    "ge_sample",
    "ge_sampler_last_error",
    "ge_sampler_max_top_k",
    "ge_sample_noalloc",
)


class SampleParams(ctypes.Structure):
    _fields_ = [
        ("temperature", ctypes.c_float),
        ("top_k", ctypes.c_uint32),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("softcap", ctypes.c_float),
        ("repetition_penalty", ctypes.c_float),
    ]


class SampleArgs(ctypes.Structure):
    _fields_ = [
        ("logits", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("rows", ctypes.c_int32),
        ("vocab", ctypes.c_int32),
        ("row_stride", ctypes.c_int64),
        ("params", SampleParams),
        ("row_params", ctypes.c_void_p),
        ("history", ctypes.c_void_p),
        ("history_offsets", ctypes.c_void_p),
        ("ring", ctypes.c_void_p),
        ("ring_len", ctypes.c_void_p),
        ("ring_capacity", ctypes.c_int32),
        ("uniforms", ctypes.c_void_p),
        ("tokens_out", ctypes.c_void_p),
        ("probs_out", ctypes.c_void_p),
        ("flags_out", ctypes.c_void_p),
        ("stop_tokens", ctypes.c_void_p),
        ("n_stop", ctypes.c_int32),
        ("stop_mode", ctypes.c_int32),
        ("done", ctypes.c_void_p),
    ]


class SamplerError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{message} (status {code})")
        self.code = code


_lib = None


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the HIP library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"{path} is missing: build it with `make -C gemmaedge_amd` (no CPU fallback exists)")
    L = ctypes.CDLL(path)
    L.ge_sampler_available.restype = ctypes.c_int
    L.ge_sampler_available.argtypes = []
    L.ge_sampler_create.restype = ctypes.c_int
    L.ge_sampler_create.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.POINTER(ctypes.c_void_p)]
    L.ge_sampler_destroy.restype = None
    L.ge_sampler_destroy.argtypes = [ctypes.c_void_p]
    L.ge_sample.restype = ctypes.c_int
    L.ge_sample.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(SampleArgs)]
    L.ge_sampler_last_error.restype = ctypes.c_char_p
    L.ge_sampler_last_error.argtypes = []
    L.ge_sampler_max_top_k.restype = ctypes.c_int
    L.ge_sampler_max_top_k.argtypes = []
    L.ge_sample_noalloc.restype = ctypes.c_int
    L.ge_sample_noalloc.argtypes = [ctypes.c_void_p, ctypes.POINTER(SampleArgs)]
    _lib = L
    return L


def last_error() -> str:
    return load_library().ge_sampler_last_error().decode()


def available() -> bool:
    return bool(load_library().ge_sampler_available())


def max_top_k() -> int:
    return int(load_library().ge_sampler_max_top_k())


# A decimal floating-point literal (what strtof reads, without hex, inf or nan).
_DECIMAL = re.compile(r"[+-]?(?:[0-9]+\.?[0-9]*|\.[0-9]+)(?:[eE][+-]?[0-9]+)?")


@dataclass
class SamplingConfig:
    """include/gemmaedge/generation.h:55-61, plus softcap / penalty (defaults = reference)."""

    temperature: float = 1.0
    top_k: int = 64
    top_p: float = 0.95
    min_p: float = 0.0
    seed: int = 0
    softcap: float = 0.0
    repetition_penalty: float = 1.0

    def params(self) -> SampleParams:
        return SampleParams(self.temperature, self.top_k, self.top_p, self.min_p, self.softcap,
                            self.repetition_penalty)

    # Environment variables of include/gemmaedge/sampling_env.h (field, type).
    ENV = {
        "GEMMAEDGE_TEMPERATURE": ("temperature", float),
        "GEMMAEDGE_TOP_K": ("top_k", int),
        "GEMMAEDGE_TOP_P": ("top_p", float),
        "GEMMAEDGE_MIN_P": ("min_p", float),
        "GEMMAEDGE_SEED": ("seed", int),
        "GEMMAEDGE_SOFTCAP": ("softcap", float),
        "GEMMAEDGE_REPETITION_PENALTY": ("repetition_penalty", float),
    }

    @classmethod
    def from_env(cls, base: "SamplingConfig | None" = None, environ=None) -> "SamplingConfig":
        """A copy of ``base`` (default: the reference defaults) with the fields
        the environment sets; unset, empty or malformed values are ignored,
        as the reference's CLI ignores a malformed GEMMAEDGE_EXPERT_CACHE_GB
        (src/main.cpp:109-115). Same rules as sampling_env.h: decimal floats
        that are finite as float32, top_k within uint32, seed within uint64,
        integers without sign; spaces and tabs around a value are allowed."""
        env = os.environ if environ is None else environ
        out = dataclasses.replace(base) if base is not None else cls()
        for name, (field, typ) in cls.ENV.items():
            text = (env.get(name) or "").strip(" \t")
            if not text:
                continue
            if typ is float:
                if not _DECIMAL.fullmatch(text):
                    continue
                try:
                    v = struct.unpack("<f", struct.pack("<f", float(text)))[0]
                except OverflowError:
                    continue
                if math.isfinite(v):
                    setattr(out, field, v)
            elif text.isascii() and text.isdigit():
                v = int(text)
                if v <= (2**32 - 1 if field == "top_k" else 2**64 - 1):
                    setattr(out, field, v)
        return out


def _ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


class Sampler:
    """Owns one ge_sampler handle (workspaces preallocated for max_rows x max_vocab)."""

    def __init__(self, max_rows: int, max_vocab: int, max_history: int = 0, device: int = 0):
        L = load_library()
        h = ctypes.c_void_p()
        rc = L.ge_sampler_create(device, max_rows, max_vocab, max_history, ctypes.byref(h))
        if rc != GE_OK:
            raise SamplerError(rc, last_error())
        self._h = h
        self.device = device
        self.max_rows = max_rows
        self.max_vocab = max_vocab

    def close(self):
        if getattr(self, "_h", None):
            load_library().ge_sampler_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def sample_raw(self, args: SampleArgs, stream=None) -> int:
        """Call ge_sample with prepared args; returns the status code."""
        s = ctypes.c_void_p(stream if isinstance(stream, int) else
                            (stream.cuda_stream if stream is not None else None))
        return load_library().ge_sample(self._h, s, ctypes.byref(args))

    def sample(self, logits, config: SamplingConfig | Sequence[SamplingConfig], uniforms=None,
               history=None, history_offsets=None, ring=None, ring_len=None, stream=None,
               tokens=None, probs=None, flags=None, row_params=None, stop_tokens=None,
               stop_mode=GE_STOP_AFTER_PUSH, done=None):
        """Sample one token per row of a [rows, vocab] (or [vocab]) device tensor.

        ``logits`` is float32 or bfloat16 on the GPU; ``uniforms`` float32 [rows];
        ``history`` int32 flat ids with ``history_offsets`` int32 [rows+1], or
        ``ring``/``ring_len`` for the device ring. ``stop_tokens`` (int32 device
        tensor) and ``done`` (int32 [rows] device tensor) enable the device-side
        stop check (see ge_sample_args). Returns (tokens, probs, flags).
        """
        import torch

        if logits.dim() == 1:
            logits = logits.unsqueeze(0)
        rows, vocab = logits.shape
        if vocab == 0:
            raise ValueError("cannot sample empty logits")
        if logits.stride(1) != 1:
            raise ValueError("logits rows must be contiguous")
        dt = {torch.float32: GE_DTYPE_F32, torch.bfloat16: GE_DTYPE_BF16}.get(logits.dtype)
        if dt is None:
            raise ValueError(f"unsupported logits dtype {logits.dtype}")
        dev = logits.device
        if stream is None:
            stream = torch.cuda.current_stream(dev)
        elif isinstance(stream, int):
            stream = torch.cuda.ExternalStream(stream, device=dev)
        # Buffers made here are allocated on the launch stream: the caching
        # allocator then keeps a block that is dropped while the kernel still
        # reads or writes it (row_params below) from being reused before the
        # stream has passed that point.
        with torch.cuda.stream(stream):
            if tokens is None:
                tokens = torch.empty(rows, dtype=torch.int32, device=dev)
            if probs is None:
                probs = torch.empty(rows, dtype=torch.float32, device=dev)
            if flags is None:
                flags = torch.empty(rows, dtype=torch.int32, device=dev)
        a = SampleArgs()
        a.logits = logits.data_ptr()
        a.dtype = dt
        a.rows = rows
        a.vocab = vocab
        # A size-1 leading dimension may carry any stride; rows must not overlap.
        a.row_stride = vocab if rows == 1 else logits.stride(0)
        if a.row_stride < vocab:
            raise ValueError("logits rows overlap (row stride < vocab)")
        if isinstance(config, SamplingConfig):
            a.params = config.params()
        else:
            a.params = config[0].params()
            if row_params is None:
                arr = (SampleParams * rows)(*[c.params() for c in config])
                with torch.cuda.stream(stream):
                    row_params = torch.frombuffer(bytearray(arr), dtype=torch.uint8).to(dev)
        a.row_params = _ptr(row_params)
        a.history = _ptr(history)
        a.history_offsets = _ptr(history_offsets)
        a.ring = _ptr(ring)
        a.ring_len = _ptr(ring_len)
        a.ring_capacity = 0 if ring is None else ring.shape[-1]
        a.uniforms = _ptr(uniforms)
        a.tokens_out = _ptr(tokens)
        a.probs_out = _ptr(probs)
        a.flags_out = _ptr(flags)
        a.stop_tokens = _ptr(stop_tokens)
        a.n_stop = 0 if stop_tokens is None else stop_tokens.numel()
        a.stop_mode = stop_mode
        a.done = _ptr(done)
        rc = self.sample_raw(a, stream)
        if rc != GE_OK:
            raise SamplerError(rc, last_error())
        return tokens, probs, flags
