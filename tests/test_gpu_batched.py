"""Batched (MFMA) step engine parity through the C ABI: sessions of more than 8 rows (independent
streams, each with its own encoder output and token sequence, or rows sharing one encoder), and
beam-size sessions forced onto the batched engine with W4H_ENGINE=wide (reorder, decode drivers).

Contract: per-step logits within max-abs 1e-2 of the oracle (fp32 activations as f16 hi/lo MFMA
operands, f16 weights, f16 KV declared), argmax bit-exact wherever the oracle's top-2 margin
exceeds that tolerance.
"""

import numpy as np
import pytest

from whisper4j_amd import synth

pytestmark = pytest.mark.gpu
TOL = 1e-2


def say(*a):
    print("[gpu-batched]", *a, flush=True)


# 80 encoder frames give one cross-attention key chunk per (encoder, head); 300 frames give three
# (chunks of at most 128 keys), whose (max, sum, value) partials k_w_cmerge merges: 10 rows on one
# encoder (two row groups of 8 and 2) and 4 rows with their own encoders.  Sessions of fewer than 5
# rows at d < 768 would run on the persistent kernel, so the 4-row case sets W4H_ENGINE=wide.
# Sessions of at most 16 rows at d in {384, 512, 768, 1024} run whole-K GEMMs with the residual,
# LayerNorm and GELU inside them, and rows sharing one encoder there run the matrix-core
# cross-attention on the transposed V copy.  mode "split" runs a case on the split-K GEMMs and
# separate kernels instead (W4H_WIDE_FUSE=0), which 20 and 32 rows and d = 1280 always use; mode
# "layerwise" projects the cross K/V (and the transposed V) with the per-layer kernel
# (W4H_XKV_LAYERWISE=1) instead of the all-layer GEMM.
@pytest.mark.parametrize("d,heads,n_rows,n_enc,wtype,a_ctx,mode", [(384, 6, 12, 12, "f16", 80, ""), (512, 8, 20, 20, "f16", 80, ""),
                                                                   (1280, 20, 32, 32, "f16", 80, ""), (1024, 16, 16, 16, "q8_0", 80, ""),
                                                                   (768, 12, 10, 1, "f16", 80, ""), (384, 6, 10, 1, "f16", 300, ""),
                                                                   (384, 6, 4, 4, "f16", 300, ""), (512, 8, 6, 1, "f16", 300, ""),
                                                                   (1024, 16, 5, 1, "q8_0", 300, ""), (768, 12, 10, 1, "f16", 80, "split"),
                                                                   (1024, 16, 16, 16, "q8_0", 80, "split"), (512, 8, 6, 1, "f16", 300, "layerwise")])
def test_batched_streams_forced(gpu, orc, monkeypatch, d, heads, n_rows, n_enc, wtype, a_ctx, mode):
    dims = synth.Dims(n_vocab=1200, n_text_ctx=48, n_text_state=d, n_text_head=heads, n_text_layer=2, n_audio_ctx=a_ctx)
    if n_rows < 5:
        monkeypatch.setenv("W4H_ENGINE", "wide")
    if mode == "split":
        monkeypatch.setenv("W4H_WIDE_FUSE", "0")
    if mode == "layerwise":
        monkeypatch.setenv("W4H_XKV_LAYERWISE", "1")
    say(f"d={d} heads={heads} rows={n_rows} encoders={n_enc} {wtype} frames={a_ctx} {mode}")
    T = synth.make_decoder(dims, seed=41, wtype=wtype, ln_random=True)
    xas = [synth.encoder_output(dims, 41, stream=e) for e in range(n_enc)]
    n_forced = 10
    prompts = [[1 + r, 2, 3] for r in range(n_rows)]
    forced = [synth.forced_tokens(n_forced, 41 + r, high=dims.n_vocab - 1) for r in range(n_rows)]
    om = orc.Model(dims, T)
    refs = [om.forced(xas[r if n_enc > 1 else 0], prompts[r], forced[r], want_logits=True) for r in range(n_rows)]
    m = gpu.Model.from_tensors(dims, T)
    s = m.session(n_rows=n_rows, n_encoders=n_enc)
    for e in range(n_enc):
        s.set_encoder(xas[e], enc=e)
    seqs = [prompts[r] + list(forced[r]) for r in range(n_rows)]
    worst, agree, covered = 0.0, 0, 0
    for i in range(len(seqs[0])):
        res, lg = s.step([seqs[r][i] for r in range(n_rows)], want_logits=True, topk=2)
        j = i - (len(prompts[0]) - 1)
        if j < 0:
            continue
        for r in range(n_rows):
            ref = refs[r]
            worst = max(worst, float(np.abs(lg[r] - ref["logits"][j]).max()))
            if ref["max"][j] - ref["second"][j] > TOL:
                covered += 1
                agree += int(res[r].argmax == ref["argmax"][j])
                assert res[r].topk_ids[0] == ref["argmax"][j]
    s.close()
    m.close()
    say("max-abs", worst, "argmax agree", agree, "/", covered)
    assert worst <= TOL
    assert agree == covered and covered > 0


def test_batched_run_greedy_feedback(gpu, monkeypatch):
    """run() with greedy feedback equals step-by-step decoding that feeds back each argmax."""
    dims = synth.Dims(n_vocab=900, n_text_ctx=40, n_text_state=512, n_text_head=8, n_text_layer=2, n_audio_ctx=64)
    T = synth.make_decoder(dims, seed=42)
    n = 12
    xas = [synth.encoder_output(dims, 42, stream=e) for e in range(n)]
    m = gpu.Model.from_tensors(dims, T)
    s = m.session(n_rows=n, n_encoders=n)
    for e in range(n):
        s.set_encoder(xas[e], enc=e)
    first = list(range(5, 5 + n))
    g = s.run(first, forced=None, n_steps=8, topk=3)
    s.reset(0)
    toks = first
    for i in range(8):
        res = s.step(toks, topk=3)
        for r in range(n):
            assert res[r].argmax == g[i][r].argmax
            assert res[r].topk_ids == g[i][r].topk_ids
            assert abs(res[r].logsumexp - g[i][r].logsumexp) < 1e-4
        toks = [x.argmax for x in res]
    s.close()
    m.close()


def test_batched_reorder_gather(gpu, orc, monkeypatch):
    """Beam-size session on the batched engine: row r after reorder(parent) continues parent[r]."""
    monkeypatch.setenv("W4H_ENGINE", "wide")
    dims = synth.Dims(n_vocab=1000, n_text_ctx=64, n_text_state=384, n_text_head=6, n_text_layer=2, n_audio_ctx=50)
    T = synth.make_decoder(dims, seed=43, ln_random=True)
    xa = synth.encoder_output(dims, 43)
    m = gpu.Model.from_tensors(dims, T)
    s = m.session(n_rows=3)
    s.set_encoder(xa)
    hist = [[1, 2], [3, 4], [5, 6]]
    for i in range(2):
        s.step([h[i] for h in hist])
    s.reorder([2, 0, 2])
    hist = [hist[2], hist[0], hist[2]]
    _, lg = s.step([9, 9, 8], want_logits=True)
    s.close()
    m.close()
    om = orc.Model(dims, T)
    for r, nxt in enumerate([9, 9, 8]):
        ref = om.forward(hist[r] + [nxt], xa)[-1]
        assert np.abs(lg[r] - ref).max() <= TOL


def test_batched_beam_driver(gpu, orc, monkeypatch):
    """The beam-5 decode driver on the batched engine against the oracle's beam search."""
    monkeypatch.setenv("W4H_ENGINE", "wide")
    dims = synth.Dims(n_vocab=1000, n_text_ctx=64, n_text_state=384, n_text_head=6, n_text_layer=2, n_audio_ctx=50)
    T = synth.make_decoder(dims, seed=44, ln_random=True)
    xa = synth.encoder_output(dims, 44)
    om = orc.Model(dims, T)
    m = gpu.Model.from_tensors(dims, T)
    sup = [1, 2, 3, 220, 500]
    bdec = gpu.WhisperDecoder(m, beam_size=5)
    b = bdec.decode_beam(xa, [10, 11, 12], 999, 15, sup, beam_size=5)
    ob = om.decode_beam(xa, [10, 11, 12], eot=999, max_tokens=15, suppress=sup, beam=5)
    assert b.tokens == ob["tokens"]
    assert b.avg_logprob == pytest.approx(ob["avg_logprob"], abs=1e-3)
    bdec.close()
    m.close()


def _session_script(gpu, dims, T, xas, n):
    """Runs of different lengths, greedy feedback, a logits request, a suppress mask and a reorder
    on one batched session; returns every result."""
    m = gpu.Model.from_tensors(dims, T)
    s = m.session(n_rows=n, n_encoders=len(xas))
    for e, xa in enumerate(xas):
        s.set_encoder(xa, enc=e)
    out = []
    first = list(range(3, 3 + n))
    forced = [[(7 * i + r) % dims.n_vocab for r in range(n)] for i in range(4)]
    out.append(s.run(first, forced=forced, n_steps=5, topk=3))
    res, lg = s.step(list(range(20, 20 + n)), want_logits=True, topk=2)
    out.append(res)
    out.append(lg)
    out.append(s.run(first, forced=None, n_steps=6, topk=1))
    s.set_suppress([1, 2, 3, 50])
    s.reorder([(r + 1) % n for r in range(n)])
    res, lg = s.step(list(range(40, 40 + n)), want_logits=True, topk=4)
    out.append(res)
    out.append(lg)
    s.close()
    m.close()
    return out


def _flatten(results):
    flat = []
    for item in results:
        if isinstance(item, np.ndarray):
            flat.append(item)
        else:
            for x in item:
                for r in (x if isinstance(x, list) else [x]):
                    flat.append((r.argmax, r.max_logit, r.logsumexp, r.raw_logsumexp, tuple(r.topk_ids), tuple(r.topk_logits)))
    return flat


def test_batched_graph_replay_matches_eager(gpu, monkeypatch):
    """The captured step, replayed for every step of a run (with eager work and synchronisations
    between runs), gives bit-identical results to launching every kernel of every step."""
    dims = synth.Dims(n_vocab=1100, n_text_ctx=40, n_text_state=512, n_text_head=8, n_text_layer=2, n_audio_ctx=64)
    T = synth.make_decoder(dims, seed=45, ln_random=True)
    n = 10
    xas = [synth.encoder_output(dims, 45, stream=e) for e in range(n)]
    monkeypatch.setenv("W4H_GRAPH", "0")
    eager = _flatten(_session_script(gpu, dims, T, xas, n))
    monkeypatch.setenv("W4H_GRAPH", "1")
    graph = _flatten(_session_script(gpu, dims, T, xas, n))
    assert len(eager) == len(graph)
    for a, b in zip(eager, graph):
        if isinstance(a, np.ndarray):
            np.testing.assert_array_equal(a, b)
        else:
            assert a == b


@pytest.mark.parametrize("beam,max_tokens,ts_begin,eot", [(5, 45, -1, 999), (5, 20, 901, 900), (3, 40, -1, 999),
                                                          (2, 70, 901, 900)])
def test_device_beam_search_matches_oracle(gpu, orc, monkeypatch, beam, max_tokens, ts_begin, eot):
    """Beam search run on the device (batched session: candidate sort, finished list, n-gram and
    timestamp masks and the slot-table reorder in k_w_beam), over more than one 32-step launch,
    against the oracle's beam search: same tokens, avg log-prob within 1e-3."""
    monkeypatch.setenv("W4H_ENGINE", "wide")
    dims = synth.Dims(n_vocab=1000, n_text_ctx=96, n_text_state=384, n_text_head=6, n_text_layer=2, n_audio_ctx=50)
    T = synth.make_decoder(dims, seed=46 + beam, ln_random=True)
    xa = synth.encoder_output(dims, 46 + beam)
    om = orc.Model(dims, T)
    m = gpu.Model.from_tensors(dims, T)
    sup = [1, 2, 3, 220]
    dec = gpu.WhisperDecoder(m, beam_size=beam, max_ctx=dims.n_text_ctx)
    for _ in range(2):  # a second search on the same session starts from a clean state
        b = dec.decode_beam(xa, [10, 11, 12], eot, max_tokens, sup, timestamp_begin=ts_begin, beam_size=beam)
        ob = om.decode_beam(xa, [10, 11, 12], eot=eot, max_tokens=max_tokens, suppress=sup, ts_begin=ts_begin, beam=beam)
        say(f"beam {beam} max {max_tokens} ts {ts_begin}: {len(b.tokens)} tokens")
        assert b.tokens == ob["tokens"]
        assert b.avg_logprob == pytest.approx(ob["avg_logprob"], abs=1e-3)
    dec.close()
    m.close()

