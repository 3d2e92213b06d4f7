"""Decoder-step parity: the persistent HIP step kernel through the C ABI against the oracle.

Contract (stated per test): per-step logits within max-abs 1e-2 of the oracle (fp32 activations,
f16 KV declared), and argmax / top-k token ids bit-exact wherever the oracle's top-2 margin
exceeds that tolerance.
"""

import numpy as np
import pytest

from whisper4j_amd import synth

pytestmark = pytest.mark.gpu
TOL = 1e-2
TINY = synth.Dims(n_vocab=1000, n_text_ctx=64, n_text_state=128, n_text_head=2, n_text_layer=2, n_audio_ctx=50)


def say(*a):
    print("[gpu-dec]", *a, flush=True)


def make(dims, seed, wtype="f16", ln_random=True):
    return synth.make_decoder(dims, seed=seed, wtype=wtype, ln_random=ln_random)


def gpu_forced_logits(gpu, dims, T, xa, prompt, forced, n_rows=1):
    m = gpu.Model.from_tensors(dims, T)
    s = m.session(n_rows=n_rows)
    s.set_encoder(xa)
    rows = []
    for i, tok in enumerate(list(prompt) + list(forced)):
        res, lg = s.step([tok] * n_rows, want_logits=True, topk=2)
        if i >= len(prompt) - 1:
            rows.append((res, lg))
    s.close()
    m.close()
    return rows


def check_rows(rows, ref, tol=TOL):
    """rows[i] = (results, logits[n_rows][V]) ; ref = oracle.forced dict (logits rows)."""
    worst, agree, covered = 0.0, 0, 0
    for i, (res, lg) in enumerate(rows):
        rl = ref["logits"][i]
        for r in range(lg.shape[0]):
            worst = max(worst, float(np.abs(lg[r] - rl).max()))
            if ref["max"][i] - ref["second"][i] > tol:
                covered += 1
                agree += int(res[r].argmax == ref["argmax"][i])
    return worst, agree, covered


def test_tiny_forced_logits(gpu, orc):
    say("tiny forced sweep f16")
    T = make(TINY, 21)
    xa = synth.encoder_output(TINY, 21)
    prompt, forced = [1, 2, 3, 4], synth.forced_tokens(40, 21, high=TINY.n_vocab - 1)
    ref = orc.Model(TINY, T).forced(xa, prompt, forced, want_logits=True)
    rows = gpu_forced_logits(gpu, TINY, T, xa, prompt, forced)
    worst, agree, covered = check_rows(rows, ref)
    say("max-abs", worst, "argmax agree", agree, "/", covered)
    assert worst <= TOL
    assert agree == covered and covered > 0


def test_tiny_q8_0(gpu, orc):
    say("tiny forced sweep q8_0")
    dims = synth.Dims(n_vocab=700, n_text_ctx=40, n_text_state=256, n_text_head=4, n_text_layer=2, n_audio_ctx=64)
    T = make(dims, 22, wtype="q8_0")
    xa = synth.encoder_output(dims, 22)
    prompt, forced = [5, 6], synth.forced_tokens(20, 22, high=dims.n_vocab - 1)
    ref = orc.Model(dims, T).forced(xa, prompt, forced, want_logits=True)
    worst, agree, covered = check_rows(gpu_forced_logits(gpu, dims, T, xa, prompt, forced), ref)
    say("max-abs", worst, "argmax agree", agree, "/", covered)
    assert worst <= TOL and agree == covered


def test_run_matches_steps_and_greedy_feedback(gpu):
    say("run vs step")
    T = make(TINY, 23)
    xa = synth.encoder_output(TINY, 23)
    m = gpu.Model.from_tensors(TINY, T)
    s = m.session()
    s.set_encoder(xa)
    forced = synth.forced_tokens(12, 23, high=TINY.n_vocab - 1)
    out_run = s.run([7], forced=forced[:11], n_steps=12, topk=3)
    s.reset(0)
    toks = [7] + list(forced[:11])
    for i, t in enumerate(toks):
        r = s.step([t], topk=3)[0]
        assert r.argmax == out_run[i][0].argmax
        assert r.topk_ids == out_run[i][0].topk_ids
        assert abs(r.logsumexp - out_run[i][0].logsumexp) < 1e-4
    # greedy feedback: each step consumes the previous argmax
    s.reset(0)
    g = s.run([7], forced=None, n_steps=10)
    s.reset(0)
    tok = 7
    for i in range(10):
        r = s.step([tok])[0]
        assert r.argmax == g[i][0].argmax
        tok = r.argmax
    s.close()
    m.close()


def test_base_en_full_context_sweep(gpu, orc):
    """base.en shape: 4-token prefix then 444 teacher-forced steps to the 448-token context."""
    dims = synth.SHAPES["base.en"]
    say("base.en 444-step sweep: building weights")
    T = make(dims, 0, ln_random=False)
    xa = synth.encoder_output(dims, 0)
    prompt = list(synth.BENCH_PREFIX)
    forced = synth.forced_tokens(444, 0)
    m = gpu.Model.from_tensors(dims, T)
    s = m.session()
    s.set_encoder(xa)
    say("base.en: gpu prefill + run")
    s.run([prompt[0]], forced=prompt[1:3], n_steps=3)
    out = s.run([prompt[3]], forced=forced[:443], n_steps=444, topk=2)
    assert s.kv_len == 447
    # the last forced token completes the 448-position context
    out_last = s.step([forced[443]], topk=2)
    assert s.kv_len == 448
    s.close()
    m.close()
    say("base.en: oracle sweep")
    ref = orc.Model(dims, T).forced(xa, prompt, forced)
    gam = np.array([o[0].argmax for o in out] + [out_last[0].argmax])
    gmax = np.array([o[0].max_logit for o in out] + [out_last[0].max_logit])
    glse = np.array([o[0].logsumexp for o in out] + [out_last[0].logsumexp])
    margin = ref["max"] - ref["second"]
    covered = margin > TOL
    say("base.en: margin>tol coverage", covered.mean(), "max|dmax|", np.abs(gmax - ref["max"]).max(),
        "max|dlse|", np.abs(glse - ref["lse"]).max())
    assert np.abs(gmax - ref["max"]).max() <= TOL
    assert np.abs(glse - ref["lse"]).max() <= TOL
    np.testing.assert_array_equal(gam[covered], ref["argmax"][covered])


def test_multistream_rows(gpu, orc):
    say("3 independent streams")
    dims = TINY
    T = make(dims, 24)
    xas = [synth.encoder_output(dims, 24, stream=i) for i in range(3)]
    m = gpu.Model.from_tensors(dims, T)
    s = m.session(n_rows=3, n_encoders=3)
    for i in range(3):
        s.set_encoder(xas[i], enc=i)
    toks = np.array([[1, 2, 3], [4, 5, 6], [7, 8, 9], [10, 11, 12], [13, 14, 15]], np.int32)
    lgs = []
    for t in toks:
        _, lg = s.step(t, want_logits=True)
        lgs.append(lg)
    s.close()
    m.close()
    om = orc.Model(dims, T)
    for r in range(3):
        ref = om.forward(toks[:, r], xas[r])
        got = np.stack([lg[r] for lg in lgs])
        assert np.abs(got - ref).max() <= TOL


def test_beam_reorder_gather(gpu, orc):
    """Row r after reorder(parent) continues parent[r]'s history."""
    say("reorder")
    T = make(TINY, 25)
    xa = synth.encoder_output(TINY, 25)
    m = gpu.Model.from_tensors(TINY, T)
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
    om = orc.Model(TINY, T)
    for r, nxt in enumerate([9, 9, 8]):
        ref = om.forward(hist[r] + [nxt], xa)[-1]
        assert np.abs(lg[r] - ref).max() <= TOL


def test_decode_drivers_match_oracle(gpu, orc):
    say("decode / decode_beam vs oracle")
    T = make(TINY, 26)
    xa = synth.encoder_output(TINY, 26)
    om = orc.Model(TINY, T)
    m = gpu.Model.from_tensors(TINY, T)
    sup = [1, 2, 3, 220, 500]
    dec = gpu.WhisperDecoder(m, beam_size=1)
    g = dec.decode(xa, [10, 11, 12], 999, 20, sup, no_speech_token=998)
    og = om.decode(xa, [10, 11, 12], eot=999, max_tokens=20, suppress=sup, no_speech=998)
    assert g.tokens == og["tokens"]
    assert g.avg_logprob == pytest.approx(og["avg_logprob"], abs=1e-3)
    assert g.no_speech_prob == pytest.approx(og["no_speech_prob"], abs=1e-4)
    assert g.compression_ratio == pytest.approx(og["compression_ratio"], rel=1e-6)
    ts = dec.decode(xa, [10, 11], 900, 10, sup, timestamp_begin=901)
    ots = om.decode(xa, [10, 11], eot=900, max_tokens=10, suppress=sup, ts_begin=901)
    assert ts.tokens == ots["tokens"]
    dec.close()
    bdec = gpu.WhisperDecoder(m, beam_size=5)
    b = bdec.decode_beam(xa, [10, 11, 12], 999, 15, sup, beam_size=5)
    ob = om.decode_beam(xa, [10, 11, 12], eot=999, max_tokens=15, suppress=sup, beam=5)
    assert b.tokens == ob["tokens"]
    assert b.avg_logprob == pytest.approx(ob["avg_logprob"], abs=1e-3)
    bdec.close()
    m.close()


def test_session_errors(gpu):
    say("error paths")
    T = make(TINY, 27)
    m = gpu.Model.from_tensors(TINY, T)
    s = m.session(max_ctx=4)
    s.set_encoder(synth.encoder_output(TINY, 27))
    with pytest.raises(gpu.W4HError) as e:
        s.step([TINY.n_vocab])
    assert e.value.code == -1
    s.run([1], forced=[2, 3, 4], n_steps=4)
    with pytest.raises(gpu.W4HError) as e:
        s.step([1])
    assert e.value.code == -8
    s.close()
    # a destroyed model refuses new sessions (IllegalStateException after close, WhisperModel.java:81-91)
    # while sessions created before keep working until they are destroyed
    import ctypes

    from whisper4j_amd import _lib

    s2 = m.session()
    s2.set_encoder(synth.encoder_output(TINY, 27))
    h = m._h
    m.close()
    out = ctypes.c_void_p()
    rc = gpu.lib().w4h_session_create(h, ctypes.byref(_lib.SessionDesc(1, 1, 16)), ctypes.byref(out))
    assert rc == _lib.W4H_ERR_CLOSED
    assert s2.step([3])[0].argmax >= 0
    s2.close()


@pytest.mark.parametrize("wtype,frames", [("f16", 300), ("q8_0", 300), ("f16", 129)])
def test_cross_kv_projection_frame_tiles(gpu, orc, wtype, frames):
    """The cross-attention K/V projection (MFMA GEMM, 128 encoder frames per workgroup) over several
    frame tiles with a partial last one: forced-decode logits within 1e-2 of the oracle; the
    device-memory entry point gives logits bit-identical to the host-memory one and refuses a host
    pointer."""
    from whisper4j_amd.device import DeviceArray

    dims = synth.Dims(n_vocab=800, n_text_ctx=32, n_text_state=256, n_text_head=4, n_text_layer=2,
                      n_audio_ctx=frames)
    say(f"cross K/V projection: {frames} frames, {wtype}")
    T = make(dims, 51, wtype=wtype)
    xa = synth.encoder_output(dims, 51)
    prompt, forced = [1, 2, 3], synth.forced_tokens(8, 51, high=dims.n_vocab - 1)
    ref = orc.Model(dims, T).forced(xa, prompt, forced, want_logits=True)
    m = gpu.Model.from_tensors(dims, T)
    out = {}
    for how in ("host", "device"):
        s = m.session()
        if how == "host":
            s.set_encoder(xa)
        else:
            xd = DeviceArray(np.asarray(xa, dtype=np.float32))
            s.set_encoder_device(xd.address)
            xd.close()
            with pytest.raises(gpu.W4HError) as e:
                s.set_encoder_device(xa.ctypes.data)
            assert e.value.code == -1
        lgs = []
        for i, tok in enumerate(prompt + list(forced)):
            _, lg = s.step([tok], want_logits=True)
            if i >= len(prompt) - 1:
                lgs.append(lg[0].copy())
        out[how] = np.array(lgs)
        s.close()
    m.close()
    worst = float(np.abs(out["host"] - ref["logits"][:len(out["host"])]).max())
    say("max-abs", worst)
    assert worst <= TOL
    np.testing.assert_array_equal(out["host"], out["device"])


def _ngram_blocks(tokens):
    """Steps of a greedy decode at which the 3/4-gram rule masks at least one token."""
    n = 0
    for j in range(1, len(tokens) + 1):
        h = tokens[:j]
        hit = any(h[i:i + 2] == h[-2:] for i in range(len(h) - 2)) or any(h[i:i + 3] == h[-3:] for i in range(len(h) - 3))
        n += int(len(h) >= 3 and hit)
    return n


@pytest.mark.parametrize("ts_begin,eot,max_tokens,max_ctx", [(-1, 399, 80, 96), (301, 300, 60, 96), (-1, 399, 80, 40)])
def test_greedy_decode_rules_on_device(gpu, orc, monkeypatch, ts_begin, eot, max_tokens, max_ctx):
    """Greedy decode of a one-row session with the n-gram and timestamp rules applied by the step
    kernel (one launch that ends at the end token): tokens and avg log-prob bit-identical to the
    host-driven loop (one step call per token, rules on the host), and tokens equal to the oracle's
    decode.  With a self-KV of 40 positions the device run stops at the capacity and the host loop
    reports the capacity error exactly as it does alone."""
    dims = synth.Dims(n_vocab=400, n_text_ctx=96, n_text_state=128, n_text_head=2, n_text_layer=2, n_audio_ctx=50)
    T = make(dims, 61)
    xa = synth.encoder_output(dims, 61)
    sup = [1, 2, 3, 220 % dims.n_vocab]
    prompt = [10, 11, 12]
    m = gpu.Model.from_tensors(dims, T)
    res = {}
    for mode in ("1", "0"):
        monkeypatch.setenv("W4H_DEVICE_RULES", mode)
        dec = gpu.WhisperDecoder(m, beam_size=1, max_ctx=max_ctx)
        try:
            res[mode] = dec.decode(xa, prompt, eot, max_tokens, sup, timestamp_begin=ts_begin)
        except gpu.W4HError as e:
            res[mode] = e.code
        dec.close()
    m.close()
    if max_ctx < len(prompt) + max_tokens:
        assert res["1"] == res["0"] == -8  # W4H_ERR_CAPACITY
        return
    dev, host = res["1"], res["0"]
    assert dev.tokens == host.tokens
    assert dev.avg_logprob == host.avg_logprob
    og = orc.Model(dims, T).decode(xa, prompt, eot=eot, max_tokens=max_tokens, suppress=sup, ts_begin=ts_begin)
    blocks = _ngram_blocks(list(og["tokens"]))
    say(f"greedy rules ts={ts_begin}: {len(dev.tokens)} tokens, n-gram rule active at {blocks} steps")
    assert dev.tokens == og["tokens"]
    assert dev.avg_logprob == pytest.approx(og["avg_logprob"], abs=1e-3)
    if ts_begin < 0:
        assert blocks > 0
    else:
        assert any(t >= ts_begin for t in dev.tokens)


@pytest.mark.parametrize("d,heads,wtype", [(768, 12, "f16"), (512, 8, "q8_0"), (1024, 16, "q8_0")])
def test_greedy_decode_rules_on_device_variants(gpu, orc, monkeypatch, d, heads, wtype):
    """The device decode rules in the other one-row step kernels (three register rounds for
    d = 768, q8_0 weights, streamed rows for d = 1024): timestamp rules on, tokens and average
    log-probability bit-identical to the host-driven loop, tokens equal to the oracle's decode."""
    dims = synth.Dims(n_vocab=500, n_text_ctx=64, n_text_state=d, n_text_head=heads, n_text_layer=2, n_audio_ctx=40)
    T = make(dims, 62, wtype=wtype)
    xa = synth.encoder_output(dims, 62)
    sup = [1, 2, 3]
    prompt, eot, tsb = [10, 11, 12], 400, 401
    m = gpu.Model.from_tensors(dims, T)
    res = {}
    for mode in ("1", "0"):
        monkeypatch.setenv("W4H_DEVICE_RULES", mode)
        dec = gpu.WhisperDecoder(m, beam_size=1, max_ctx=dims.n_text_ctx)
        res[mode] = dec.decode(xa, prompt, eot, 40, sup, timestamp_begin=tsb)
        dec.close()
    m.close()
    assert res["1"].tokens == res["0"].tokens
    assert res["1"].avg_logprob == res["0"].avg_logprob
    og = orc.Model(dims, T).decode(xa, prompt, eot=eot, max_tokens=40, suppress=sup, ts_begin=tsb)
    say(f"greedy rules d={d} {wtype}: {len(res['1'].tokens)} tokens")
    assert res["1"].tokens == og["tokens"]
    assert res["1"].avg_logprob == pytest.approx(og["avg_logprob"], abs=1e-3)


# ---- temperature sampling and the fallback driver ------------------------------------------------

FB_DIMS = synth.Dims(n_vocab=600, n_text_ctx=320, n_text_state=128, n_text_head=2, n_text_layer=2, n_audio_ctx=50)


def _fb_model(seed=71):
    T = make(FB_DIMS, seed)
    xa = synth.encoder_output(FB_DIMS, seed)
    return T, xa


def _draw_margins(orc, om, xa, prompt, eot, suppress, temperature, seed, tokens, n_steps):
    """Relative distance of each sampling draw of the oracle's decode from the nearest bucket edge of
    the cumulative weights (0 where a 1e-4 change of the weights could move it to a neighbouring id)."""
    lg = om.forced(xa, prompt, np.array(tokens[: n_steps - 1], np.int32), want_logits=True)["logits"]
    us = orc.rng_uniform(seed, n_steps)
    out = []
    for i in range(n_steps):
        row = lg[i]
        if i == 0:
            row = orc.suppress_blank(row, eot)
        row = orc.apply_suppress(row, suppress)
        row = orc.ngram_block(orc.ngram_block(row, tokens[:i], 3), tokens[:i], 4)
        w = np.exp(((row - row.max()) / np.float32(temperature)).astype(np.float64)).astype(np.float32).astype(np.float64)
        cum = np.cumsum(w)
        r = us[i] * cum[-1]
        k = int(np.searchsorted(cum, r))
        lo = cum[k - 1] if k > 0 else 0.0
        out.append(min(r - lo, cum[k] - r) / cum[-1])
    return out


@pytest.mark.parametrize("temperature,seed", [(0.4, 3), (1.0, 11)])
def test_sampled_decode_matches_oracle(gpu, orc, temperature, seed):
    """WhisperDecoder.decode at T > 0 (sample, main/nn/WhisperDecoder.java:576-598) with the seeded
    draw: tokens equal to the oracle's decode with the same seed up to the first draw that lies within
    1e-4 (relative) of a bucket edge of the cumulative weights (logits agree to ~1e-4, so such a draw
    may legitimately pick a neighbour); average log-probability within 1e-3 when the decodes agree."""
    T, xa = _fb_model()
    om = orc.Model(FB_DIMS, T)
    m = gpu.Model.from_tensors(FB_DIMS, T)
    dec = gpu.WhisperDecoder(m, beam_size=1)
    prompt, eot, sup = [10, 11, 12], 599, [1, 2]
    g = dec.decode(xa, prompt, eot, 60, sup, temperature=temperature, seed=seed)
    o = om.decode(xa, prompt, eot=eot, max_tokens=60, suppress=sup, temperature=temperature, seed=seed)
    dec.close()
    m.close()
    n = len(o["tokens"]) + (1 if len(o["tokens"]) < 60 else 0)
    marg = _draw_margins(orc, om, xa, prompt, eot, sup, temperature, seed, list(o["tokens"]), n)
    first = next((i for i in range(min(len(g.tokens), len(o["tokens"]))) if g.tokens[i] != o["tokens"][i]), None)
    say(f"T={temperature} seed={seed}: {len(g.tokens)} tokens (oracle {len(o['tokens'])}), first difference {first}, "
        f"smallest draw margin {min(marg):.2e}")
    if first is None:
        assert g.tokens == o["tokens"]
        assert g.avg_logprob == pytest.approx(o["avg_logprob"], abs=1e-3)
        assert g.temperature == pytest.approx(temperature)
    else:
        assert min(marg[: first + 1]) < 1e-4, f"decodes part at step {first} with every draw margin >= 1e-4"


@pytest.mark.parametrize("temperature,seed,ts_begin,rows", [(0.6, 7, -1, 1), (1.0, 21, 500, 1), (0.4, 9, -1, 3)])
def test_device_sampling_equals_host_sampling(gpu, monkeypatch, temperature, seed, ts_begin, rows):
    """A decode at T > 0 samples every step after the first on the device (w4h_sample.hip, chained
    after one-step launches of the step kernel, the token handed over in device memory).  Against the
    host loop that fetches each row and samples it (W4H_DEVICE_SAMPLE=0) on the same session, inputs
    and seed: identical tokens and average log-probability within 1e-9 (both draw from the device's
    logits with the same generator; the rules and the suppress list run on both sides)."""
    T, xa = _fb_model(seed=73)
    m = gpu.Model.from_tensors(FB_DIMS, T)
    dec = gpu.WhisperDecoder(m, beam_size=rows)
    prompt, eot, sup = [10, 11, 12], 599, [1, 2]
    res = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("W4H_DEVICE_SAMPLE", mode)
        res[mode] = dec.decode(xa, prompt, eot, 120, sup, temperature=temperature, seed=seed, timestamp_begin=ts_begin)
    dec.close()
    m.close()
    h, d = res["0"], res["1"]
    say(f"T={temperature} seed={seed} ts={ts_begin} rows={rows}: host {len(h.tokens)} tokens avg {h.avg_logprob:.6f}, "
        f"device {len(d.tokens)} tokens avg {d.avg_logprob:.6f}")
    assert d.tokens == h.tokens
    assert abs(d.avg_logprob - h.avg_logprob) <= 1e-6
    assert len(d.tokens) > 5


@pytest.mark.parametrize("d,heads,wtype,temperature,seed,ts_begin", [(128, 2, "f16", 0.6, 7, -1), (128, 2, "f16", 1.0, 21, 500),
                                                                   (768, 12, "f16", 0.8, 3, -1), (256, 4, "q8_0", 0.7, 5, 500)])
def test_sampling_in_launch_equals_chain(gpu, monkeypatch, d, heads, wtype, temperature, seed, ts_begin):
    """A sampled run on a one-row session draws its tokens inside one launch of the step kernel (the
    grid's phase after the logits: row maximum, per-workgroup weight sums, the crossing range, the
    token), instead of one-step launches chained with the masking and sampling kernels
    (W4H_SAMPLE_IN_LAUNCH=0).  Same session, inputs and seed: identical tokens and average
    log-probability within 1e-9 (the two sum the weights in different orders, which moves only the last
    bits of a double).  Covers the three sampled instances of the step kernel: f16 with two and three
    register rounds (d = 128, 768) and q8_0."""
    dims = synth.Dims(n_vocab=600, n_text_ctx=320, n_text_state=d, n_text_head=heads, n_text_layer=2, n_audio_ctx=50)
    T = make(dims, 73, wtype=wtype)
    xa = synth.encoder_output(dims, 73)
    m = gpu.Model.from_tensors(dims, T)
    dec = gpu.WhisperDecoder(m, beam_size=1)
    prompt, eot, sup = [10, 11, 12], 599, [1, 2]
    res = {}
    monkeypatch.setenv("W4H_DEVICE_SAMPLE", "1")
    for mode in ("0", "2"):  # 2: the in-launch path without falling back to the chain
        monkeypatch.setenv("W4H_SAMPLE_IN_LAUNCH", mode)
        res[mode] = dec.decode(xa, prompt, eot, 120, sup, temperature=temperature, seed=seed, timestamp_begin=ts_begin)
    dec.close()
    m.close()
    c, i = res["0"], res["2"]
    say(f"d={d} {wtype} T={temperature} seed={seed} ts={ts_begin}: chain {len(c.tokens)} tokens avg {c.avg_logprob:.9f}, "
        f"in-launch {len(i.tokens)} tokens avg {i.avg_logprob:.9f}")
    assert i.tokens == c.tokens
    assert abs(i.avg_logprob - c.avg_logprob) <= 1e-9
    assert len(i.tokens) > 5


@pytest.mark.parametrize("shape,wtype", [("base.en", "f16"), ("small", "f16"), ("medium", "q8_0")])
def test_sampling_in_launch_full_vocab(gpu, monkeypatch, shape, wtype):
    """The in-launch sampler at the real vocabulary (51864-51865 ids, ~203 per workgroup range, one
    per thread) and full depth, against the launch chain on the same session, inputs and seed:
    identical tokens, average log-probability within 1e-9.  base.en and small f16 (two and three
    register rounds), medium q8_0; 1500 encoder frames, the multilingual prompt, 48 tokens at T = 0.7
    with the end token suppressed so both run to the end."""
    dims = synth.SHAPES[shape]
    say(f"in-launch sampler, {shape} {wtype}: building weights")
    T = synth.make_decoder(dims, seed=3, wtype=wtype)
    xa = synth.encoder_output(dims, 3)
    m = gpu.Model.from_tensors(dims, T)
    dec = gpu.WhisperDecoder(m, beam_size=1)
    prompt, eot = list(synth.BENCH_PREFIX), synth.EOT_MULTILINGUAL
    res = {}
    monkeypatch.setenv("W4H_DEVICE_SAMPLE", "1")
    for mode in ("0", "2"):  # 2: the in-launch path without falling back to the chain
        monkeypatch.setenv("W4H_SAMPLE_IN_LAUNCH", mode)
        res[mode] = dec.decode(xa, prompt, eot, 48, [eot], temperature=0.7, seed=11)
    dec.close()
    m.close()
    c, i = res["0"], res["2"]
    say(f"{shape}: chain {len(c.tokens)} tokens avg {c.avg_logprob:.9f}, in-launch {len(i.tokens)} tokens avg {i.avg_logprob:.9f}")
    assert len(i.tokens) == 48
    assert i.tokens == c.tokens
    assert abs(i.avg_logprob - c.avg_logprob) <= 1e-9


@pytest.mark.parametrize("beam", [1, 3])
def test_decode_with_fallback_matches_oracle(gpu, orc, beam):
    """WhisperDecoder.decodeWithFallback (main/nn/WhisperDecoder.java:119-149) on a model whose greedy
    decode compresses better than 2.4 (a fixed logit bias favours six ids), so needsFallback holds at
    T = 0 and the loop decodes the sampled temperatures (seed + i) before it returns: the device
    driver's result (tokens, temperature, average log-probability, compression ratio) equals the
    oracle's driver on the same inputs; beam 3 runs the T = 0 decode as beam search.  Each sampled
    temperature's decode is also compared on its own with the oracle's."""
    T, xa = _fb_model()
    bias = np.zeros(FB_DIMS.n_vocab, np.float32)
    bias[100:106] = 8.0
    om = orc.Model(FB_DIMS, T)
    om.set_logit_bias(bias)
    m = gpu.Model.from_tensors(FB_DIMS, T)
    dec = gpu.WhisperDecoder(m, beam_size=beam)
    dec.set_logit_bias(bias)
    prompt, eot, sup, n, seed = [10, 11, 12], 599, [1, 2], 250, 5
    o0 = om.decode(xa, prompt, eot=eot, max_tokens=n, suppress=sup) if beam == 1 else \
        om.decode_beam(xa, prompt, eot=eot, max_tokens=n, suppress=sup, beam=beam)
    say(f"fallback beam={beam}: oracle T=0 compression {o0['compression_ratio']:.3f} avg {o0['avg_logprob']:.3f}")
    assert o0["compression_ratio"] > 2.4  # the loop goes past T = 0
    g = dec.decode_with_fallback(xa, prompt, eot, n, sup, beam_size=beam, seed=seed)
    o = om.decode_with_fallback(xa, prompt, eot=eot, max_tokens=n, suppress=sup, beam=beam, seed=seed)
    say(f"fallback beam={beam}: device T={g.temperature} {len(g.tokens)} tokens avg {g.avg_logprob:.4f}; "
        f"oracle T={o['temperature']} avg {o['avg_logprob']:.4f}")
    assert g.tokens == o["tokens"]
    assert g.temperature == pytest.approx(o["temperature"])
    assert g.avg_logprob == pytest.approx(o["avg_logprob"], abs=1e-3)
    assert g.compression_ratio == pytest.approx(o["compression_ratio"], rel=1e-6)
    if beam == 1:
        for i, t in enumerate([0.2, 0.4, 0.6, 0.8, 1.0], start=1):
            gs = dec.decode(xa, prompt, eot, n, sup, temperature=t, seed=seed + i)
            os_ = om.decode(xa, prompt, eot=eot, max_tokens=n, suppress=sup, temperature=t, seed=seed + i)
            say(f"fallback T={t}: device avg {gs.avg_logprob:.4f} oracle {os_['avg_logprob']:.4f} "
                f"equal tokens {gs.tokens == os_['tokens']}")
            assert gs.tokens == os_["tokens"]
    dec.close()
    m.close()
