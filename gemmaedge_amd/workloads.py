"""Seeded synthetic inputs for the benchmark configurations C1-C5.

There are no model weights offline, so logits are drawn from the distributions
the configurations name (normal with peaks, log-Zipf, near-uniform bf16).
Numbers come from numpy's Philox counter-based generator with a recorded seed.
Uniforms come from std::mt19937_64(seed) through generate_canonical<float, 24>,
which is what the reference's decode loop feeds its sampler
(src/main.cpp:133, src/generation.cpp:118-119); ``MT19937_64`` below restates
that engine (Matsumoto & Nishimura, 2000) so the Python side draws the same
stream as the C++ drop-in.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

VOCAB = 262144


class MT19937_64:
    """64-bit Mersenne Twister with the std::mt19937_64 parameters
    (the template arguments of the reference's engine type)."""

    N, M = 312, 156
    MATRIX_A = 0xB5026F5AA96619E9
    UPPER = 0xFFFFFFFF80000000
    LOWER = 0x7FFFFFFF
    MASK = (1 << 64) - 1

    def __init__(self, seed: int = 5489):
        mt = [0] * self.N
        mt[0] = seed & self.MASK
        for i in range(1, self.N):
            mt[i] = (6364136223846793005 * (mt[i - 1] ^ (mt[i - 1] >> 62)) + i) & self.MASK
        self.mt = mt
        self.i = self.N

    def _twist(self):
        mt = self.mt
        for i in range(self.N):
            x = (mt[i] & self.UPPER) | (mt[(i + 1) % self.N] & self.LOWER)
            xa = x >> 1
            if x & 1:
                xa ^= self.MATRIX_A
            mt[i] = mt[(i + self.M) % self.N] ^ xa
        self.i = 0

    def __call__(self) -> int:
        if self.i >= self.N:
            self._twist()
        x = self.mt[self.i]
        self.i += 1
        x ^= (x >> 29) & 0x5555555555555555
        x ^= (x << 17) & 0x71D67FFFEDA60000
        x ^= (x << 37) & 0xFFF7EEE000000000
        x ^= x >> 43
        return x & self.MASK


def canonical_float(x: int) -> float:
    """generate_canonical<float, 24> for one 64-bit engine output
    (libstdc++ random.tcc:3345-3380): float(x) / 2^64 with round-to-nearest-even
    conversion, clamped below 1."""
    if x == 0:
        return 0.0
    nbits = x.bit_length()
    shift = max(nbits - 24, 0)
    q = x >> shift
    if shift:
        rem = x & ((1 << shift) - 1)
        half = 1 << (shift - 1)
        if rem > half or (rem == half and (q & 1)):
            q += 1
    # q < 2^24 and the scale is a power of two in the normal range: exact.
    val = np.float32(q) * np.float32(2.0 ** (shift - 64))
    if val >= np.float32(1.0):
        val = np.nextafter(np.float32(1.0), np.float32(0.0))
    return float(val)


def mt_uniforms(seed: int, n: int) -> np.ndarray:
    eng = MT19937_64(seed)
    return np.array([canonical_float(eng()) for _ in range(n)], dtype=np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16 bit patterns (finite inputs)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


@dataclass
class Workload:
    name: str
    logits: np.ndarray                 # [rows, vocab] float32, or uint16 bf16 bits
    dtype: str                         # "f32" or "bf16"
    params: dict                       # temperature, top_k, top_p, min_p, softcap, repetition_penalty
    history: np.ndarray                # int32 flat
    offsets: np.ndarray                # int32 [rows + 1]
    uniforms: np.ndarray               # float32 [rows]
    seed: int = 0
    notes: dict = field(default_factory=dict)

    @property
    def rows(self) -> int:
        return self.logits.shape[0]

    @property
    def vocab(self) -> int:
        return self.logits.shape[1]

    def bytes_per_row(self) -> float:
        """Algorithmic HBM bytes per row: V*s + 4*H + 12 (logits, history,
        uniform in, token and prob out)."""
        s = 2 if self.dtype == "bf16" else 4
        h = (self.offsets[-1] - self.offsets[0]) / max(self.rows, 1)
        return self.vocab * s + 4 * h + 12


def _rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.Philox(seed))


def _histories(rng, rows, h, vocab):
    hist = rng.integers(0, vocab, size=rows * h, dtype=np.int64).astype(np.int32)
    offsets = (np.arange(rows + 1, dtype=np.int64) * h).astype(np.int32)
    return hist, offsets


def c1(seed: int = 1, vocab: int = VOCAB, greedy: bool = False) -> Workload:
    """Single row, N(0,3) + 16 peaks of +8; softcap 30, T 1.0, k 64, p 0.95,
    penalty 1.1 over 128 ids; one uniform from mt19937_64(seed)."""
    rng = _rng(seed)
    x = (rng.standard_normal(vocab, dtype=np.float32) * np.float32(3.0)).astype(np.float32)
    peaks = rng.choice(vocab, size=min(16, vocab), replace=False)
    x[peaks] += np.float32(8.0)
    hist, offsets = _histories(rng, 1, 128, vocab)
    p = dict(temperature=0.0 if greedy else 1.0, top_k=64, top_p=0.95, min_p=0.0,
             softcap=30.0, repetition_penalty=1.1)
    return Workload("C1-greedy" if greedy else "C1", x[None, :], "f32", p, hist, offsets,
                    mt_uniforms(seed, 1), seed)


def c2(seed: int = 2, rows: int = 64, vocab: int = VOCAB) -> Workload:
    """Batch 64, N(0,3) with 8-32 peaks of +U(6,10) per row; softcap 30, T 0.7,
    k 40, p 0.9, penalty 1.15 over 2048 ids per row (duplicates)."""
    rng = _rng(seed)
    x = (rng.standard_normal((rows, vocab), dtype=np.float32) * np.float32(3.0)).astype(np.float32)
    for r in range(rows):
        n = int(rng.integers(8, 33))
        idx = rng.choice(vocab, size=min(n, vocab), replace=False)
        x[r, idx] += rng.uniform(6.0, 10.0, size=idx.size).astype(np.float32)
    hist, offsets = _histories(rng, rows, 2048, vocab)
    p = dict(temperature=0.7, top_k=40, top_p=0.9, min_p=0.0, softcap=30.0,
             repetition_penalty=1.15)
    return Workload("C2", x, "f32", p, hist, offsets, mt_uniforms(seed, rows), seed)


def c3(seed: int = 3, rows: int = 256, vocab: int = VOCAB) -> Workload:
    """Batch 256, log(Zipf(1.1)) over a seeded permutation + N(0,0.5); T 1.0,
    k 1024, p 0.99, penalty 1.05 over 512 ids; softcap 30 (model default)."""
    rng = _rng(seed)
    ranks = np.arange(1, vocab + 1, dtype=np.float64)
    base = (-1.1 * np.log(ranks)).astype(np.float32)
    x = np.empty((rows, vocab), np.float32)
    for r in range(rows):
        perm = rng.permutation(vocab)
        x[r, perm] = base
        x[r] += (rng.standard_normal(vocab, dtype=np.float32) * np.float32(0.5))
    hist, offsets = _histories(rng, rows, 512, vocab)
    p = dict(temperature=1.0, top_k=1024, top_p=0.99, min_p=0.0, softcap=30.0,
             repetition_penalty=1.05)
    return Workload("C3", x, "f32", p, hist, offsets, mt_uniforms(seed, rows), seed)


def c4(seed: int = 4, rows: int = 512, vocab: int = VOCAB, f32: bool = False) -> Workload:
    """Batch 512, bf16 N(0,0.1) (RNE from f32); top-k off, p 0.9, T 1.3, no
    penalty; softcap 30 (model default). f32=True keeps the f32 logits (the
    same rows before rounding): the f32 full-order path."""
    rng = _rng(seed)
    x = (rng.standard_normal((rows, vocab), dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    hist = np.zeros(0, np.int32)
    offsets = np.zeros(rows + 1, np.int32)
    p = dict(temperature=1.3, top_k=0, top_p=0.9, min_p=0.0, softcap=30.0,
             repetition_penalty=1.0)
    if f32:
        return Workload("C4-f32", x, "f32", p, hist, offsets, mt_uniforms(seed, rows), seed)
    return Workload("C4", f32_to_bf16_bits(x), "bf16", p, hist, offsets, mt_uniforms(seed, rows), seed)


def c5_steps(seed: int = 5, steps: int = 1024, vocab: int = VOCAB) -> Workload:
    """Decode sweep: `steps` consecutive fp32 rows N(0,3) + 16 peaks; history
    grows on the device by each sampled token (ring of 8192); penalty 1.1,
    k 64, p 0.95, T 1.0; softcap 30."""
    rng = _rng(seed)
    x = (rng.standard_normal((steps, vocab), dtype=np.float32) * np.float32(3.0)).astype(np.float32)
    for r in range(steps):
        idx = rng.choice(vocab, size=min(16, vocab), replace=False)
        x[r, idx] += np.float32(8.0)
    p = dict(temperature=1.0, top_k=64, top_p=0.95, min_p=0.0, softcap=30.0,
             repetition_penalty=1.1)
    w = Workload("C5", x, "f32", p, np.zeros(0, np.int32), np.zeros(steps + 1, np.int32),
                 mt_uniforms(seed, steps), seed)
    w.notes["ring_capacity"] = 8192
    return w


CONFIGS = {"C1": c1, "C2": c2, "C3": c3, "C4": c4, "C5": c5_steps}


def to_device(w: Workload, device="cuda"):
    """Copy a workload's inputs to the GPU: (logits, history, offsets, uniforms);
    bf16 logits become a torch.bfloat16 view of the same bits."""
    import torch

    if w.dtype == "bf16":
        logits = torch.from_numpy(np.ascontiguousarray(w.logits).view(np.int16)).to(device).view(torch.bfloat16)
    else:
        logits = torch.from_numpy(np.ascontiguousarray(w.logits)).to(device)
    hist = torch.from_numpy(w.history.astype(np.int32)).to(device) if w.history.size else None
    offs = torch.from_numpy(w.offsets.astype(np.int32)).to(device) if w.history.size else None
    uni = torch.from_numpy(w.uniforms.astype(np.float32)).to(device)
    return logits, hist, offs, uni
