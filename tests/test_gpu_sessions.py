"""Batched multi-session decode on the device: several sessions share one
ge_sample launch captured in a HIP graph, each with its own device history
ring, parameters, stop check and done flag (the decode loop of
Gemma4Session::generate, src/generation.cpp:452-469, with the stop tokens of
include/gemmaedge/generation.h:66, for N sessions at once). Every replay is
checked against the CPU oracle given each row's explicit history.

Also: the full-order path under a wrapping ring (the history bitmap must be
cleared from the ids the call read, not from the ring after the append),
rows with padding (row_stride > vocab), and rows that are done on entry."""
import ctypes

import numpy as np
import pytest

import ge_oracle as O
from gemmaedge_amd import workloads as W

pytestmark = pytest.mark.gpu

STOP = (1, 106)  # <eos>, <turn|> (include/gemmaedge/generation.h:66)


def _peaked_steps(seed, steps, rows, vocab, peaks=24, lift=5.0, scale=1.0, stop_at=None):
    """[steps, rows, vocab] f32: N(0, scale) noise plus a fixed set of peaks per
    row (so sampled tokens recur and the penalty history matters). stop_at maps
    (row, step) -> stop token lifted far above everything at that step."""
    rng = np.random.Generator(np.random.Philox(seed))
    x = (rng.standard_normal((steps, rows, vocab), dtype=np.float32) * np.float32(scale)).astype(np.float32)
    for r in range(rows):
        idx = rng.choice(np.arange(200, vocab), size=peaks, replace=False)
        x[:, r, idx] += np.float32(lift)
    for (r, s), tok in (stop_at or {}).items():
        x[s, r, tok] = np.float32(60.0)
    return x


def _row_params(torch, params):
    from gemmaedge_amd import sampler as S

    arr = (S.SampleParams * len(params))(*[S.SamplingConfig(**p).params() for p in params])
    return torch.frombuffer(bytearray(arr), dtype=torch.uint8).cuda()


def _run_session(label, mode, params, stop_at, cap, steps, seed, shared=False, vocab=262144):
    """Captures one ge_sample over len(params) rows with a device ring, stop
    tokens and done flags, replays it `steps` times and checks every replay,
    the final ring, ring_len and done against the oracle. shared=True passes
    params[0] as the call's shared parameters (no row_params)."""
    import torch

    from gemmaedge_amd import Sampler
    from gemmaedge_amd import sampler as S

    rows = len(params)
    stop_mode = S.GE_STOP_AFTER_PUSH if mode == "after_push" else S.GE_STOP_BEFORE_PUSH
    x = _peaked_steps(seed, steps, rows, vocab, stop_at=stop_at)
    u_all = W.mt_uniforms(seed + 20, steps * rows).reshape(steps, rows)
    print(f"[sessions] {label} {mode}: rows={rows} V={vocab} cap={cap} steps={steps} shared={shared}", flush=True)

    s = Sampler(max_rows=rows, max_vocab=vocab, max_history=cap)
    logits = torch.empty((rows, vocab), dtype=torch.float32, device="cuda")
    uni = torch.empty(rows, dtype=torch.float32, device="cuda")
    ring = torch.zeros((rows, cap), dtype=torch.int32, device="cuda")
    ring_len = torch.zeros(rows, dtype=torch.int32, device="cuda")
    done = torch.zeros(rows, dtype=torch.int32, device="cuda")
    stops = torch.tensor(STOP, dtype=torch.int32, device="cuda")
    tokens = torch.empty(rows, dtype=torch.int32, device="cuda")
    probs = torch.empty(rows, dtype=torch.float32, device="cuda")
    flags = torch.empty(rows, dtype=torch.int32, device="cuda")
    a = S.SampleArgs()
    a.logits, a.dtype, a.rows, a.vocab, a.row_stride = logits.data_ptr(), S.GE_DTYPE_F32, rows, vocab, vocab
    a.params = S.SamplingConfig(**params[0]).params()
    rp = None if shared else _row_params(torch, params)
    if rp is not None:
        a.row_params = rp.data_ptr()
    a.ring, a.ring_len, a.ring_capacity = ring.data_ptr(), ring_len.data_ptr(), cap
    a.uniforms, a.tokens_out, a.probs_out, a.flags_out = (uni.data_ptr(), tokens.data_ptr(),
                                                          probs.data_ptr(), flags.data_ptr())
    a.stop_tokens, a.n_stop, a.stop_mode, a.done = stops.data_ptr(), len(STOP), stop_mode, done.data_ptr()
    lib = S.load_library()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            rc = lib.ge_sample(s._h, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream), ctypes.byref(a))
    assert rc == 0, S.last_error()
    torch.cuda.synchronize()
    ring.zero_()
    ring_len.zero_()
    done.zero_()

    pushed = [[] for _ in range(rows)]
    finished = [False] * rows
    stopped_rows = set()
    oparams = [O.make_params(**p) for p in params]
    for i in range(steps):
        logits.copy_(torch.from_numpy(x[i]))
        uni.copy_(torch.from_numpy(u_all[i]))
        g.replay()
        _ = (logits * 2.0).sum()  # unrelated eager work between replays
        torch.cuda.synchronize()
        got_t = tokens.cpu().numpy()
        got_p = probs.cpu().numpy().view(np.uint32)
        got_f = flags.cpu().numpy()
        live = [r for r in range(rows) if not finished[r]]
        if live:
            hs = [np.array(pushed[r][-cap:], np.int32) for r in live]
            offs = np.concatenate([[0], np.cumsum([h.size for h in hs])]).astype(np.int32)
            ora = O.run(x[i, live], [oparams[r] for r in live],
                        history=np.concatenate(hs) if offs[-1] else np.zeros(0, np.int32), offsets=offs,
                        uniforms=u_all[i, live], nthreads=4)
        for j, r in enumerate(live):
            assert got_t[r] == ora.tokens[j], f"step {i} row {r}: gpu {got_t[r]} oracle {ora.tokens[j]}"
            assert got_p[r] == ora.probs.view(np.uint32)[j], f"step {i} row {r} prob"
            is_stop = int(ora.tokens[j]) in STOP
            assert bool(got_f[r] & S.GE_FLAG_STOP) == is_stop, f"step {i} row {r} stop flag"
            if not (is_stop and stop_mode == S.GE_STOP_BEFORE_PUSH):
                pushed[r].append(int(ora.tokens[j]))
            if is_stop:
                finished[r] = True
                stopped_rows.add(r)
        for r in range(rows):
            if r not in live:
                assert got_t[r] == -1 and got_f[r] == S.GE_FLAG_DONE, f"step {i} row {r} done"
    assert stopped_rows >= {r for (r, _) in stop_at}
    np.testing.assert_array_equal(ring_len.cpu().numpy(), [len(p) for p in pushed])
    np.testing.assert_array_equal(done.cpu().numpy(), [1 if f else 0 for f in finished])
    rg = ring.cpu().numpy()
    for r in range(rows):
        n = len(pushed[r])
        want = np.zeros(cap, np.int32)
        for t in range(n):
            want[t % cap] = pushed[r][t]
        np.testing.assert_array_equal(rg[r], want, err_msg=f"ring row {r}")
    s.close()


@pytest.mark.parametrize("mode", ["after_push", "before_push"])
def test_multi_session_ring_graph_with_stop(mode):
    base = dict(softcap=30.0, min_p=0.0)
    params = [dict(base, temperature=1.0, top_k=64, top_p=0.95, repetition_penalty=1.1),
              dict(base, temperature=0.7, top_k=40, top_p=0.9, repetition_penalty=1.15),
              dict(base, temperature=0.0, top_k=64, top_p=0.95, repetition_penalty=1.3),  # greedy
              dict(base, temperature=1.3, top_k=512, top_p=0.99, repetition_penalty=1.05),
              dict(base, temperature=1.0, top_k=1, top_p=1.0, repetition_penalty=1.0),
              dict(base, temperature=0.9, top_k=200, top_p=0.8, repetition_penalty=0.9),   # r < 1
              dict(base, temperature=1.0, top_k=64, top_p=0.95, repetition_penalty=1.1, min_p=0.05),
              dict(base, temperature=1.2, top_k=1024, top_p=0.95, repetition_penalty=1.2)]
    stop_at = {(1, 9): 106, (4, 17): 1, (6, 30): 106}
    _run_session("per-row", mode, params, stop_at, cap=24, steps=44, seed=11)


@pytest.mark.parametrize("mode", ["after_push", "before_push"])
@pytest.mark.parametrize("rows", [3, 12])
def test_greedy_sessions_shared_params(mode, rows):
    """Shared parameters with temperature 0: every row takes the greedy kernel,
    with its polled last-chunk merge at 3 rows (64 chunks each, all resident)
    and its ticket merge at 12. The penalty over the wrapping ring makes each
    row's argmax move as its own tokens recur; the device ring append, the
    stop check and the done rows are the greedy kernel's own."""
    p = dict(temperature=0.0, top_k=64, top_p=0.95, min_p=0.0, softcap=30.0, repetition_penalty=1.3)
    stop_at = {(1, 7): 106, (rows - 1, 15): 1}
    if rows > 4:
        stop_at[(5, 22)] = 106
    _run_session("greedy", mode, [p] * rows, stop_at, cap=8, steps=30, seed=17 + rows, shared=True)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_full_order_ring_wraps(dtype):
    """top_k = 0 (full-order path) with a penalty over a ring smaller than the
    step count: once the ring is full every append evicts an id whose bit in
    the path's history bitmap must be cleared, or a later call skips (bf16)
    or penalises (f32) a token that is no longer in the history."""
    import torch

    from gemmaedge_amd import Sampler
    from gemmaedge_amd import sampler as S

    rows, vocab, cap, steps = 2, 262144, 6, 22
    p = dict(temperature=1.0, top_k=0, top_p=0.9, min_p=0.0, softcap=30.0, repetition_penalty=1.15)
    x = _peaked_steps(13, steps, rows, vocab, peaks=8, lift=9.0)
    if dtype == "bf16":
        xs = W.f32_to_bf16_bits(x)
        dev = torch.from_numpy(xs.view(np.int16)).cuda().view(torch.bfloat16)
    else:
        xs = x
        dev = torch.from_numpy(xs).cuda()
    u_all = W.mt_uniforms(37, steps * rows).reshape(steps, rows)
    print(f"[sessions] full-order ring {dtype}: rows={rows} cap={cap} steps={steps}", flush=True)
    s = Sampler(max_rows=rows, max_vocab=vocab, max_history=cap)
    ring = torch.zeros((rows, cap), dtype=torch.int32, device="cuda")
    ring_len = torch.zeros(rows, dtype=torch.int32, device="cuda")
    cfg = S.SamplingConfig(**p)
    pushed = [[] for _ in range(rows)]
    op = O.make_params(**p)
    for i in range(steps):
        uni = torch.from_numpy(u_all[i]).cuda()
        t, pr, _ = s.sample(dev[i], cfg, uniforms=uni, ring=ring, ring_len=ring_len)
        torch.cuda.synchronize()
        hs = [np.array(pushed[r][-cap:], np.int32) for r in range(rows)]
        offs = np.concatenate([[0], np.cumsum([h.size for h in hs])]).astype(np.int32)
        ora = O.run(xs[i], op, history=np.concatenate(hs) if offs[-1] else np.zeros(0, np.int32),
                    offsets=offs, uniforms=u_all[i], nthreads=2)
        np.testing.assert_array_equal(t.cpu().numpy(), ora.tokens, err_msg=f"step {i}")
        np.testing.assert_array_equal(pr.cpu().numpy().view(np.uint32), ora.probs.view(np.uint32),
                                      err_msg=f"step {i} probs")
        for r in range(rows):
            pushed[r].append(int(ora.tokens[r]))
    s.close()


@pytest.mark.parametrize("pad", [64, 3])
@pytest.mark.parametrize("case", ["select", "full_order_bf16"])
def test_padded_rows(pad, case):
    """Rows with padding after the vocabulary (row_stride > vocab), as an
    LM head with padded columns leaves them: the padding must never be read as
    logits. pad = 3 also breaks 16-byte row alignment (scalar load path)."""
    import torch

    from gemmaedge_amd import Sampler, SamplingConfig

    vocab = 262144
    if case == "select":
        w = W.c2(rows=8)
    else:
        w = W.c4(rows=8)
    rows = w.rows
    print(f"[sessions] padded {case} pad={pad}", flush=True)
    if w.dtype == "bf16":
        big = np.full((rows, vocab + pad), 0x7F7F, np.uint16)  # huge finite bf16 in the padding
        big[:, :vocab] = w.logits
        dev = torch.from_numpy(big.view(np.int16)).cuda().view(torch.bfloat16)[:, :vocab]
    else:
        big = np.full((rows, vocab + pad), 1e30, np.float32)
        big[:, :vocab] = w.logits
        dev = torch.from_numpy(big).cuda()[:, :vocab]
    assert dev.stride(0) == vocab + pad
    hist = torch.from_numpy(w.history).cuda() if w.history.size else None
    offs = torch.from_numpy(w.offsets).cuda() if w.history.size else None
    uni = torch.from_numpy(w.uniforms).cuda()
    with Sampler(max_rows=rows, max_vocab=vocab, max_history=2048) as s:
        t, p, f = s.sample(dev, SamplingConfig(**w.params), uniforms=uni, history=hist, history_offsets=offs)
        torch.cuda.synchronize()
    ora = O.run(w.logits, O.make_params(**w.params), history=w.history if w.history.size else None,
                offsets=w.offsets if w.history.size else None, uniforms=w.uniforms)
    np.testing.assert_array_equal(t.cpu().numpy(), ora.tokens)
    np.testing.assert_array_equal(p.cpu().numpy().view(np.uint32), ora.probs.view(np.uint32))


def test_done_rows_are_skipped():
    import torch

    from gemmaedge_amd import Sampler, SamplingConfig
    from gemmaedge_amd import sampler as S

    w = W.c2(rows=6)
    logits, hist, offs, uni = W.to_device(w)
    done = torch.tensor([0, 1, 0, 1, 1, 0], dtype=torch.int32, device="cuda")
    ring = torch.full((6, 4), 5, dtype=torch.int32, device="cuda")
    ring_len = torch.full((6,), 2, dtype=torch.int32, device="cuda")
    with Sampler(max_rows=6, max_vocab=w.vocab, max_history=2048) as s:
        t, p, f = s.sample(logits, SamplingConfig(**w.params), uniforms=uni, ring=ring, ring_len=ring_len,
                           done=done)
        torch.cuda.synchronize()
    hist_rows = np.tile(np.array([5, 5], np.int32), 6)
    ora = O.run(w.logits, O.make_params(**w.params), history=hist_rows,
                offsets=(np.arange(7) * 2).astype(np.int32), uniforms=w.uniforms)
    t, f = t.cpu().numpy(), f.cpu().numpy()
    for r in range(6):
        if done[r]:
            assert t[r] == -1 and f[r] == S.GE_FLAG_DONE
        else:
            assert t[r] == ora.tokens[r]
    np.testing.assert_array_equal(ring_len.cpu().numpy(), [3, 2, 3, 2, 2, 3])
    assert (done.cpu().numpy() == [0, 1, 0, 1, 1, 0]).all()
