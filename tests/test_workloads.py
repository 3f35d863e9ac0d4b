"""Synthetic inputs of the benchmark configurations (CPU)."""
import numpy as np
import torch

from gemmaedge_amd import workloads as W


def test_bf16_rounding_matches_torch():
    x = (np.random.default_rng(0).standard_normal(100000) * 3).astype(np.float32)
    ours = W.f32_to_bf16_bits(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    assert np.array_equal(W.bf16_bits_to_f32(ours), torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def test_generators_are_seeded_and_shaped():
    a, b = W.c2(rows=4, vocab=4096), W.c2(rows=4, vocab=4096)
    assert np.array_equal(a.logits, b.logits) and np.array_equal(a.history, b.history)
    assert a.logits.shape == (4, 4096) and a.logits.dtype == np.float32
    assert a.offsets.tolist() == [0, 2048, 4096, 6144, 8192]
    c4 = W.c4(rows=3, vocab=4096)
    assert c4.logits.dtype == np.uint16 and c4.dtype == "bf16" and c4.history.size == 0
    c1 = W.c1(vocab=4096)
    assert c1.rows == 1 and c1.params["top_k"] == 64 and c1.history.size == 128
    c3 = W.c3(rows=2, vocab=4096)
    assert c3.params["top_k"] == 1024


def test_bytes_per_row_formula():
    # B_row = V*s + 4*H + 12
    assert W.c2(rows=2, vocab=1024).bytes_per_row() == 1024 * 4 + 4 * 2048 + 12
    assert W.c4(rows=2, vocab=1024).bytes_per_row() == 1024 * 2 + 12
