"""The C ABI's boundary paths on the GPU: the GGML file loader, the positional clamp past the text
context, the threading contract, and the size guard of the persistent kernel's 32-bit addressing.

Contract (per test): logits of a model loaded from a GGML file bit-identical to the same tensors
uploaded from memory; logits past n_text_ctx within 1e-2 of the oracle, which clamps the positional
row as the reference does; sessions driven from two threads give results bit-identical to the same
work run one after the other.
"""

import threading

import numpy as np
import pytest

from whisper4j_amd import synth

pytestmark = pytest.mark.gpu
TOL = 1e-2


def say(*a):
    print("[gpu-boundary]", *a, flush=True)


@pytest.mark.parametrize("wtype", ["f16", "q8_0"])
def test_ggml_file_load_matches_tensor_table(gpu, tmp_path, wtype):
    """w4h_model_load_ggml (GgmlLoader.load, main/model/GgmlLoader.java:95-220) on a whisper.cpp file
    written from a tensor table gives logits bit-identical to w4h_model_create on that table."""
    dims = synth.Dims(n_vocab=700, n_text_ctx=32, n_text_state=256, n_text_head=4, n_text_layer=2, n_audio_ctx=64)
    T = synth.make_decoder(dims, seed=81, wtype=wtype, ln_random=True)
    path = str(tmp_path / f"ggml-{wtype}.bin")
    synth.write_ggml(path, dims, T, ftype=1 if wtype == "f16" else 7)
    xa = synth.encoder_output(dims, 81)
    toks = [1, 2, 3] + list(synth.forced_tokens(10, 81, high=dims.n_vocab - 1))
    got = {}
    for how in ("table", "file"):
        m = gpu.Model.from_tensors(dims, T) if how == "table" else gpu.Model.load_ggml(path)
        d = m.dims
        assert (d.n_vocab, d.n_text_ctx, d.n_text_state, d.n_text_head, d.n_text_layer, d.n_audio_ctx) == (
            700, 32, 256, 4, 2, 64)
        s = m.session()
        s.set_encoder(xa)
        got[how] = np.stack([s.step([t], want_logits=True)[1][0] for t in toks])
        s.close()
        m.close()
    say(f"ggml {wtype}: {len(toks)} steps, max |table - file| {np.abs(got['table'] - got['file']).max()}")
    np.testing.assert_array_equal(got["table"], got["file"])


@pytest.mark.parametrize("engine,n_rows", [("persistent", 1), ("wide", 5)])
def test_positional_clamp_past_context(gpu, orc, monkeypatch, engine, n_rows):
    """A self-KV larger than n_text_ctx: past the context every token takes positional row
    n_text_ctx - 1 while the cache keeps growing (offset = min(kv_len, n_ctx - seqLen),
    main/nn/WhisperDecoder.java:72).  24 steps past a 16-position context, within 1e-2 of the oracle."""
    monkeypatch.setenv("W4H_ENGINE", engine)
    dims = synth.Dims(n_vocab=500, n_text_ctx=16, n_text_state=256, n_text_head=4, n_text_layer=2, n_audio_ctx=40)
    T = synth.make_decoder(dims, seed=82, ln_random=True)
    xa = synth.encoder_output(dims, 82)
    toks = [5, 6, 7] + list(synth.forced_tokens(37, 82, high=dims.n_vocab - 1))
    om = orc.Model(dims, T)
    c = om.new_cache()
    ref = [om.forward(toks[:3], xa, c)[-1]] + [om.forward([t], xa, c)[0] for t in toks[3:]]
    assert len(c) == 40
    m = gpu.Model.from_tensors(dims, T)
    s = m.session(n_rows=n_rows, max_ctx=48)
    s.set_encoder(xa)
    rows = []
    for i, t in enumerate(toks):
        _, lg = s.step([t] * n_rows, want_logits=True)
        if i >= 2:
            rows.append(lg)
    s.close()
    m.close()
    worst = max(float(np.abs(rows[j][r] - ref[j]).max()) for j in range(len(ref)) for r in range(n_rows))
    past = max(float(np.abs(rows[j][0] - ref[j]).max()) for j in range(14, len(ref)))
    say(f"clamp {engine}: {len(ref)} rows (positions to 39 of a 16 context), max-abs {worst:.2e}, past the context {past:.2e}")
    assert worst <= TOL


def _sweep(model, dims, xa, forced, n_rows):
    s = model.session(n_rows=n_rows, max_ctx=dims.n_text_ctx)
    s.set_encoder(xa)
    s.run([1] * n_rows, forced=[[2] * n_rows, [3] * n_rows], n_steps=3)
    out = s.run([int(forced[0])] * n_rows, forced=[[int(t)] * n_rows for t in forced[1:]], n_steps=len(forced), topk=3)
    s.close()
    return [(r.argmax, r.max_logit, r.logsumexp, tuple(r.topk_ids)) for step in out for r in step]


def test_two_threads_share_one_model(gpu):
    """The threading contract (test/ConcurrencyTest.java:33-93: concurrent transcriptions equal serial
    ones): one model, sessions on two threads at once (a one-row persistent session and a six-row
    batched session on each thread, three rounds), every result bit-identical to the serial run."""
    dims = synth.Dims(n_vocab=900, n_text_ctx=64, n_text_state=384, n_text_head=6, n_text_layer=2, n_audio_ctx=60)
    T = synth.make_decoder(dims, seed=83, ln_random=True)
    m = gpu.Model.from_tensors(dims, T)
    jobs = [(synth.encoder_output(dims, 83, stream=k), synth.forced_tokens(40, 83 + k, high=dims.n_vocab - 1), rows)
            for k, rows in enumerate([1, 6, 1, 6])]
    serial = [_sweep(m, dims, *j) for j in jobs]
    results = [[None] * len(jobs) for _ in range(3)]
    errors = []

    def worker(rnd, idx):
        try:
            for k in idx:
                results[rnd][k] = _sweep(m, dims, *jobs[k])
        except Exception as e:  # reported below
            errors.append(e)

    for rnd in range(3):
        th = [threading.Thread(target=worker, args=(rnd, idx)) for idx in ([0, 1], [2, 3])]
        for t in th:
            t.start()
        for t in th:
            t.join(timeout=120)
        assert not any(t.is_alive() for t in th), "a decode thread did not finish"
    m.close()
    assert not errors, errors
    for rnd in range(3):
        for k in range(len(jobs)):
            assert results[rnd][k] == serial[k], f"round {rnd}, job {k} differs from the serial run"
    say(f"two threads: {len(jobs)} sessions x 3 rounds equal to the serial runs")


def test_persistent_kernel_size_guard(gpu, monkeypatch):
    """The persistent kernel addresses its cross-KV and self-KV through 32-bit offsets: a session whose
    cross-KV would pass 2 GiB is refused at creation (W4H_ERR_INVALID), not run with a truncated range."""
    monkeypatch.setenv("W4H_ENGINE", "persistent")
    dims = synth.Dims(n_vocab=300, n_text_ctx=64, n_text_state=1024, n_text_head=16, n_text_layer=2, n_audio_ctx=140000)
    T = synth.make_decoder(dims, seed=84)
    m = gpu.Model.from_tensors(dims, T)
    # 4 encoders x 2 layers x 16 heads x 140000 frames x 64 x 2 bytes = 2.29 GB per K and V
    with pytest.raises(gpu.W4HError) as e:
        m.session(n_rows=4, n_encoders=4, max_ctx=64)
    assert e.value.code == -1 and "2 GiB" in str(e.value)
    # the batched engine addresses the same buffers with 64-bit offsets and takes the session
    monkeypatch.setenv("W4H_ENGINE", "wide")
    s = m.session(n_rows=4, n_encoders=4, max_ctx=64)
    s.close()
    m.close()


@pytest.mark.parametrize("mode", ["greedy", "sampled", "beam"])
def test_cancel_from_another_thread(gpu, mode):
    """w4h_session_cancel (TranscriptionHandle.cancel, main/WhisperModel.java:620-633) from another
    thread while the owner thread is inside a long decode: a greedy decode running as one launch
    (decode rules on the device), a sampled decode (T = 0.5, a chain of launches) and a beam-5 search
    on the batched engine each return W4H_ERR_CANCELLED well before the uncancelled decode's time;
    calls on the cancelled session return W4H_ERR_CANCELLED at once; once cleared, the same decode on
    the same session gives the uncancelled result again."""
    import time

    dims = synth.Dims(n_vocab=2000, n_text_ctx=1024, n_text_state=256, n_text_head=4, n_text_layer=4, n_audio_ctx=64)
    T = synth.make_decoder(dims, seed=31)
    xa = synth.encoder_output(dims, 31)
    beam = 5 if mode == "beam" else 1
    prompt, eot, n = [1, 2, 3], 1999, 900 if mode != "beam" else 600
    kw = dict(temperature=0.5, seed=4) if mode == "sampled" else {}
    with gpu.Model.from_tensors(dims, T) as m:
        dec = gpu.WhisperDecoder(m, beam_size=beam, max_ctx=1024)
        run = (lambda: dec.decode_beam(xa, prompt, eot, n, [eot], beam_size=5)) if mode == "beam" else \
              (lambda: dec.decode(xa, prompt, eot, n, [eot], **kw))
        run()  # warm-up
        t0 = time.perf_counter()
        full = run()
        t_full = time.perf_counter() - t0
        assert len(full.tokens) >= n - 2
        delay = 0.2 * t_full
        th = threading.Timer(delay, lambda: dec.session.cancel(True))
        t0 = time.perf_counter()
        th.start()
        with pytest.raises(gpu.W4HError) as ei:
            run()
        t_cancel = time.perf_counter() - t0
        th.join()
        say(f"{mode}: uncancelled {t_full * 1e3:.1f} ms, cancel after {delay * 1e3:.1f} ms returned after {t_cancel * 1e3:.1f} ms")
        assert ei.value.code == -11
        assert t_cancel < 0.6 * t_full
        with pytest.raises(gpu.W4HError) as ei:
            run()
        assert ei.value.code == -11
        dec.session.cancel(False)
        again = run()
        assert again.tokens == full.tokens
        assert again.avg_logprob == full.avg_logprob
        dec.close()
