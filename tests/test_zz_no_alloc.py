"""ge_sample_noalloc (the allocation-free entry point) against ge_sample, through
the C ABI: two calls in a row on the same GPU, the second with a smaller input
(fewer rows, another dtype and parameters), each compared bit for bit (tokens,
probabilities, flags) with ge_sample on identical inputs; then the capacity
errors. The entry point has no counterpart in the reference; its output must
equal the handle path's, which the parity tests tie to the oracle."""
import ctypes

import numpy as np
import pytest

from gemmaedge_amd import workloads as W

pytestmark = pytest.mark.gpu


def _args(S, w, logits, hist, offs, uni, outs):
    a = S.SampleArgs()
    a.logits = logits.data_ptr()
    a.dtype = S.GE_DTYPE_BF16 if w.dtype == "bf16" else S.GE_DTYPE_F32
    a.rows, a.vocab, a.row_stride = w.rows, w.vocab, w.vocab
    a.params = S.SamplingConfig(**w.params).params()
    if hist is not None:
        a.history, a.history_offsets = hist.data_ptr(), offs.data_ptr()
    a.uniforms = uni.data_ptr()
    a.tokens_out, a.probs_out, a.flags_out = (t.data_ptr() for t in outs)
    return a


def _outs(torch, rows):
    return (torch.full((rows,), -7, dtype=torch.int32, device="cuda"),
            torch.zeros(rows, dtype=torch.float32, device="cuda"),
            torch.full((rows,), -7, dtype=torch.int32, device="cuda"))


def _bits(outs):
    t, p, f = (x.cpu().numpy() for x in outs)
    return t, p.view(np.uint32), f


def test_noalloc_matches_handle_path_twice():
    import torch

    from gemmaedge_amd import sampler as S

    L = S.load_library()
    c2 = W.c2()
    small = W.c2(seed=9, rows=8)
    small.logits = W.f32_to_bf16_bits(small.logits)
    small.dtype = "bf16"
    small.params = dict(temperature=1.0, top_k=1024, top_p=0.99, min_p=0.02, softcap=30.0,
                        repetition_penalty=1.05)
    s = S.Sampler(max_rows=64, max_vocab=W.VOCAB, max_history=2048)
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    for call, w in enumerate((c2, small)):
        print(f"[noalloc] call {call}: {w.name} rows={w.rows} {w.dtype} {w.params}", flush=True)
        logits, hist, offs, uni = W.to_device(w)
        ref_outs, got_outs = _outs(torch, w.rows), _outs(torch, w.rows)
        ref = _args(S, w, logits, hist, offs, uni, ref_outs)
        got = _args(S, w, logits, hist, offs, uni, got_outs)
        assert s.sample_raw(ref, stream) == 0, S.last_error()
        assert L.ge_sample_noalloc(sp, ctypes.byref(got)) == 0, S.last_error()
        torch.cuda.synchronize()
        rt, rp, rf = _bits(ref_outs)
        gt, gp, gf = _bits(got_outs)
        assert (rt >= 0).all()
        np.testing.assert_array_equal(gt, rt)
        np.testing.assert_array_equal(gp, rp)
        np.testing.assert_array_equal(gf, rf)
    s.close()


def test_noalloc_rejects_what_it_cannot_hold():
    import torch

    from gemmaedge_amd import sampler as S

    L = S.load_library()
    sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    w = W.c4(rows=4)  # top_k = 0 over V: needs the full-order workspace
    logits, hist, offs, uni = W.to_device(w)
    outs = _outs(torch, w.rows)
    a = _args(S, w, logits, hist, offs, uni, outs)
    assert L.ge_sample_noalloc(sp, ctypes.byref(a)) == S.GE_ERR_CAPACITY
    assert "full-order" in S.last_error()
    a.rows = S.GE_NOALLOC_MAX_ROWS + 1
    assert L.ge_sample_noalloc(sp, ctypes.byref(a)) == S.GE_ERR_CAPACITY
    assert "GE_NOALLOC_MAX_ROWS" in S.last_error()
    torch.cuda.synchronize()
    assert (outs[0].cpu().numpy() == -7).all()  # nothing was launched
