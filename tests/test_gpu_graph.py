"""Graph capture: one ge_sample launch captured into a HIP graph and replayed
as a decode loop would, with the history ring and its length on the device
(ge_sample_args.ring / ring_len). Every replay is checked against the oracle
given the explicit history of previously sampled tokens; eager work runs
between replays."""
import ctypes

import numpy as np
import pytest

import ge_oracle as O
from gemmaedge_amd import workloads as W

pytestmark = pytest.mark.gpu


def test_ring_history_under_graph_replay():
    import torch

    from gemmaedge_amd import Sampler
    from gemmaedge_amd import sampler as S

    steps, vocab, cap = 40, 262144, 16  # capacity below steps: the window wraps
    w = W.c5_steps(steps=steps, vocab=vocab)
    s = Sampler(max_rows=1, max_vocab=vocab, max_history=cap)
    all_logits = torch.from_numpy(w.logits).cuda()
    uni_all = torch.from_numpy(w.uniforms).cuda()
    logits = torch.empty(vocab, dtype=torch.float32, device="cuda")
    uni = torch.empty(1, dtype=torch.float32, device="cuda")
    ring = torch.zeros((1, cap), dtype=torch.int32, device="cuda")
    ring_len = torch.zeros(1, dtype=torch.int32, device="cuda")
    tokens = torch.empty(1, dtype=torch.int32, device="cuda")
    probs = torch.empty(1, dtype=torch.float32, device="cuda")
    flags = torch.empty(1, dtype=torch.int32, device="cuda")
    a = S.SampleArgs()
    a.logits, a.dtype, a.rows, a.vocab, a.row_stride = logits.data_ptr(), S.GE_DTYPE_F32, 1, vocab, vocab
    a.params = S.SamplingConfig(**w.params).params()
    a.ring, a.ring_len, a.ring_capacity = ring.data_ptr(), ring_len.data_ptr(), cap
    a.uniforms, a.tokens_out, a.probs_out, a.flags_out = (uni.data_ptr(), tokens.data_ptr(),
                                                          probs.data_ptr(), flags.data_ptr())
    lib = S.load_library()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            rc = lib.ge_sample(s._h, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
                               ctypes.byref(a))
    assert rc == 0, S.last_error()
    torch.cuda.synchronize()
    ring.zero_()
    ring_len.zero_()
    history = []
    p = O.make_params(**w.params)
    for i in range(steps):
        logits.copy_(all_logits[i])
        uni.copy_(uni_all[i:i + 1])
        g.replay()
        _ = (logits * 2.0).sum()  # unrelated eager work between replays
        torch.cuda.synchronize()
        tok = int(tokens.item())
        h = np.array(history[-cap:], np.int32)
        ora = O.run(w.logits[i:i + 1], p, history=h, offsets=np.array([0, h.size], np.int32),
                    uniforms=w.uniforms[i:i + 1], nthreads=1)
        assert tok == int(ora.tokens[0]), f"step {i}"
        assert probs.cpu().numpy().view(np.uint32)[0] == ora.probs.view(np.uint32)[0]
        history.append(tok)
    assert int(ring_len.item()) == steps
    s.close()
