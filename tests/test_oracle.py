"""Pins the oracle (a CPU restatement of whisper4j's decode path) before it is trusted as the parity reference.

Each check is either a known answer held by the reference's own tests (cited file:line, relative to
src/test/java/com/sparrowlogic/whisper4j/), an exact closed form, a brute-force float64 evaluation,
or an invariant a plausible mistake would break.
"""

import json
import os
import zlib

import numpy as np
import pytest

from tests import np_decoder
from whisper4j_amd import synth

TINY = synth.Dims(n_vocab=800, n_text_ctx=64, n_text_state=128, n_text_head=2, n_text_layer=2, n_audio_ctx=40)


# ---- known answers from the reference's unit tests (tests/golden/reference_known_answers.json) ----

def _golden():
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_known_answers.json")) as f:
        return json.load(f)


GOLDEN = _golden()


@pytest.mark.parametrize("case", GOLDEN["dot"], ids=lambda c: c["cite"])
def test_dot_known_answers(orc, case):
    assert abs(orc.dot(case["a"], case["b"]) - case["expect"]) <= case["tol"]


def test_dot_long_within_reference_bound(orc):
    # tensor/SimdOpsTest.java:52-70: 512-length dot within 0.1 of the sequential sum
    a = (np.arange(512) * 0.01).astype(np.float32)
    b = ((512 - np.arange(512)) * 0.01).astype(np.float32)
    seq = np.float32(0)
    for i in range(512):
        seq = np.float32(seq + np.float32(a[i] * b[i]))
    assert abs(orc.dot(a, b) - float(seq)) <= 0.1


@pytest.mark.parametrize("case", GOLDEN["linear"], ids=lambda c: c["cite"])
def test_linear_known_answers(orc, case):
    # Linear takes W [out][in]: y = x . W^T
    got = orc.linear(np.array(case["x"], np.float32), np.array(case["w"], np.float32))
    np.testing.assert_allclose(got, case["expect"], atol=case["tol"], rtol=0)


@pytest.mark.parametrize("case", GOLDEN["softmax"], ids=lambda c: c["cite"])
def test_softmax_known_answers(orc, case):
    np.testing.assert_allclose(orc.softmax_rows(case["x"]), case["expect"], atol=case["tol"], rtol=0)


@pytest.mark.parametrize("case", GOLDEN["softmax_row_sums"], ids=lambda c: c["cite"])
def test_softmax_row_sums(orc, case):
    np.testing.assert_allclose(orc.softmax_rows(case["x"]).sum(1), case["expect"], atol=case["tol"], rtol=0)


@pytest.mark.parametrize("case", GOLDEN["layernorm"], ids=lambda c: c["cite"])
def test_layernorm_known_answers(orc, case):
    out = orc.layernorm(np.array(case["x"], np.float32), np.array(case["gamma"], np.float32),
                        np.array(case["beta"], np.float32))
    np.testing.assert_allclose(out[:, case["columns"]], case["expect"], atol=case["tol"], rtol=0)


@pytest.mark.parametrize("case", GOLDEN["layernorm_row_mean"], ids=lambda c: c["cite"])
def test_layernorm_row_mean(orc, case):
    out = orc.layernorm(np.array(case["x"], np.float32), np.array(case["gamma"], np.float32),
                        np.array(case["beta"], np.float32))
    np.testing.assert_allclose(out.mean(1), case["expect"], atol=case["tol"], rtol=0)


@pytest.mark.parametrize("case", GOLDEN["gelu"], ids=lambda c: c["cite"])
def test_gelu_known_answers(orc, case):
    np.testing.assert_allclose(orc.gelu(np.array(case["x"], np.float32)), case["expect"], atol=case["tol"], rtol=0)


# ---- exact closed forms ---------------------------------------------------------------------

def test_f16_conversion_matches_ieee(orc):
    # widening is exact and RNE narrowing inverts it for every non-NaN half
    for h in list(range(0, 0x7C01, 97)) + list(range(0x8000, 0xFC01, 101)) + [0x7BFF, 0x0001, 0x03FF, 0x0400]:
        f = orc.f16_to_f32(h)
        assert f == float(np.array([h], np.uint16).view(np.float16)[0])
        assert orc.f32_to_f16(f) == h
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.standard_normal(2000).astype(np.float32) * 10.0 ** rng.integers(-8, 5, 2000),
                         np.array([65504, 65519.99, 65520, 1e-8, 2.0 ** -25, 2.0 ** -24 * 1.5], np.float32)])
    for x in xs.astype(np.float32):
        assert orc.f32_to_f16(float(x)) == int(np.array([x], np.float32).astype(np.float16).view(np.uint16)[0])


def test_gelu_table_against_float64(orc):
    # the table is the reference's float expression; it must sit within a few ulps of exact GELU
    t = orc.gelu_table()
    x = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float64)
    ok = np.isfinite(x) & (np.abs(x) < 60)
    x = np.where(ok, x, 0.0)
    exact = 0.5 * x * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x ** 3)))
    err = np.abs(t[ok] - exact[ok])
    assert np.all(err <= 1e-6 * np.maximum(1.0, np.abs(exact[ok])) + 1e-30)
    assert t[0] == 0.0 and t[0x3C00] == pytest.approx(0.8412, abs=1e-4)  # gelu(0), gelu(1)


def test_q8_0_dequant_closed_form(orc):
    rng = np.random.default_rng(1)
    w = rng.standard_normal((4, 64)).astype(np.float32) * 0.02
    raw = synth.quantize_q8_0(w)
    blocks = raw.reshape(-1, 34)
    d = blocks[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1)
    q = blocks[:, 2:].view(np.int8).astype(np.float32)
    expect = (q * d[:, None]).reshape(-1)
    out = orc.dequant_q8_0(raw, 256)
    np.testing.assert_array_equal(out, expect)
    # round-to-nearest quantizer: |w - q*d| <= d/2, plus the f16 rounding of d (|q| <= 127)
    amax = np.abs(w.reshape(-1, 32)).max(1, keepdims=True)
    bound = amax / 127 * (0.5 + 127 * 2.0 ** -11) * 1.001
    assert np.all(np.abs(out.reshape(-1, 32) - w.reshape(-1, 32)) <= bound)


# ---- brute force in float64 -----------------------------------------------------------------

def test_linear_error_bound(orc):
    rng = np.random.default_rng(2)
    for m, k, n in [(1, 512, 96), (3, 384, 40), (1, 2048, 16)]:
        x = rng.standard_normal((m, k)).astype(np.float32)
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        b = (rng.standard_normal(n) * 0.02).astype(np.float32)
        y = orc.linear(x, w, b)
        ref = x.astype(np.float64) @ w.T.astype(np.float64) + b
        bound = (k + 1) * 2.0 ** -24 * (np.abs(x.astype(np.float64)) @ np.abs(w.T.astype(np.float64)) + np.abs(b))
        assert np.all(np.abs(y - ref) <= bound * 1.01 + 1e-30)


def test_attention_head_brute_force(orc):
    rng = np.random.default_rng(3)
    for L in (1, 5, 300):
        q = rng.standard_normal(64).astype(np.float32)
        k = rng.standard_normal((L, 64)).astype(np.float32)
        v = rng.standard_normal((L, 64)).astype(np.float32)
        out = orc.attention_head(q, k, v, 0.125)
        s = k.astype(np.float64) @ q * 0.125
        p = np.exp(s - s.max())
        p /= p.sum()
        np.testing.assert_allclose(out, p @ v, atol=2e-5, rtol=1e-5)


def test_selection_rules(orc):
    # argmax keeps the first maximum (main/nn/WhisperDecoder.java:566-574)
    assert orc.argmax([1, 3, 3, 2]) == 1
    assert orc.argmax([-np.inf] * 4) == 0
    # topkIndices: descending, ties keep the lower index, unfilled slots stay 0
    assert orc.topk([1, 5, 5, 2, 5], 3) == [1, 2, 4]
    assert orc.topk([-np.inf, 3, -np.inf], 3) == [1, 0, 0]
    # computeLogSoftmax
    lp = orc.log_softmax(np.array([1, 2, 3], np.float32))
    np.testing.assert_allclose(lp, np.array([1, 2, 3]) - np.log(np.exp([1, 2, 3]).sum()), atol=1e-6)


def test_compression_ratio_zlib(orc):
    toks = [50364, 440, 440, 440, 1012, 50400] * 9
    raw = b"".join(int(t & 0xFFFF).to_bytes(2, "little") for t in toks)
    assert orc.compression_ratio(toks) == pytest.approx(len(raw) / len(zlib.compress(raw)), rel=1e-6)
    assert orc.compression_ratio([]) == 0.0


# ---- whole-decoder composition ----------------------------------------------------------------

@pytest.fixture(scope="module")
def tiny(orc):
    T = synth.make_decoder(TINY, seed=5, ln_random=True)
    return T, orc.Model(TINY, T), synth.encoder_output(TINY, 5)


def test_forward_matches_float64_formulation(tiny):
    T, m, xa = tiny
    toks = [3, 17, 250, 799, 0, 44, 600]
    ours = m.forward(toks, xa)
    ref = np_decoder.forward(np_decoder.weights64(T), TINY, toks, xa)
    assert np.abs(ours - ref).max() < 2e-4 * max(1.0, np.abs(ref).max())


def test_incremental_cache_equals_full_recompute(tiny):
    # the reference's own invariant (tools/generate_reference_values.py:232-257): KV-cached
    # single-token steps reproduce the rows of one full forward pass
    T, m, xa = tiny
    toks = [5, 9, 13, 200, 300, 400]
    full = m.forward(toks, xa)
    c = m.new_cache()
    rows = [m.forward(toks[:3], xa, c)[-1]]
    for t in toks[3:]:
        rows.append(m.forward([t], xa, c)[0])
    assert len(c) == len(toks)
    np.testing.assert_allclose(np.stack(rows), full[2:], atol=1e-5)


def test_positional_offset_clamp(orc):
    # offset = min(len(kv), n_ctx - seqLen) (main/nn/WhisperDecoder.java:72): past the context the
    # position stays at n_ctx-1 while the cache keeps growing
    dims = synth.Dims(n_vocab=300, n_text_ctx=6, n_text_state=64, n_text_head=1, n_text_layer=1, n_audio_ctx=8)
    T = synth.make_decoder(dims, seed=9)
    m = orc.Model(dims, T)
    xa = synth.encoder_output(dims, 9)
    c = m.new_cache()
    m.forward([1, 2], xa, c)
    for t in range(3, 10):
        m.forward([t], xa, c)
    assert len(c) == 9


def test_decode_drivers_consistent(tiny):
    T, m, xa = tiny
    sup = [1, 2, 3, 7, 220]
    g = m.decode(xa, [10, 11], eot=799, max_tokens=12, suppress=sup)
    assert not set(g["tokens"]) & set(sup)
    assert len(g["tokens"]) <= 12
    # beam 1 ranks exactly like greedy when timestamps are off
    b1 = m.decode_beam(xa, [10, 11], eot=799, max_tokens=12, suppress=sup, beam=1)
    assert b1["tokens"] == g["tokens"][: len(b1["tokens"])]
    b5 = m.decode_beam(xa, [10, 11], eot=799, max_tokens=12, suppress=sup, beam=5)
    assert 1 <= len(b5["tokens"]) <= 12 and not set(b5["tokens"]) & set(sup)
    # timestamps: first generated token is a timestamp within the first second
    ts = m.decode(xa, [10, 11], eot=700, max_tokens=6, ts_begin=701)
    assert 701 <= ts["tokens"][0] <= 751


def test_forced_sweep_records(tiny):
    T, m, xa = tiny
    f = synth.forced_tokens(6, 1, high=TINY.n_vocab - 1)
    r = m.forced(xa, [1, 2, 3], f, want_logits=True)
    lg = r["logits"]
    np.testing.assert_array_equal(r["argmax"], lg.argmax(1))
    np.testing.assert_allclose(r["lse"], np.log(np.exp(lg.astype(np.float64)).sum(1)), atol=1e-5)
