"""Kernel-level parity: each decoder building block, run through the C ABI on the GPU, against the
oracle on the same inputs.  Integer/table work is bit-exact; floating-point work is held to the
bound stated in each test."""

import math

import numpy as np
import pytest

from whisper4j_amd import synth

pytestmark = pytest.mark.gpu


def say(*a):
    print("[gpu-op]", *a, flush=True)


def test_gelu_table_bit_exact(gpu, orc):
    say("gelu over all 65536 f16 values")
    x = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    ok = ~np.isnan(x)
    y = gpu.op_gelu(x)
    t = orc.gelu_table()
    np.testing.assert_array_equal(y[ok], t[ok])
    rng = np.random.default_rng(0)
    r = (rng.standard_normal(100000) * 3).astype(np.float32)
    np.testing.assert_array_equal(gpu.op_gelu(r), orc.gelu(r))


@pytest.mark.parametrize("n", [64, 384, 512, 1280, 5120])
def test_layernorm(gpu, orc, n):
    say("layernorm n", n)
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((3, n)) * 2 + 0.5).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    b = (0.1 * rng.standard_normal(n)).astype(np.float32)
    np.testing.assert_allclose(gpu.op_layernorm(x, g, b), orc.layernorm(x, g, b), atol=2e-5, rtol=1e-5)


@pytest.mark.parametrize("m,n,k", [(1, 512, 512), (1, 1536, 512), (5, 96, 768), (8, 40, 2048), (1, 24, 5120),
                                   (1, 13, 384)])
def test_linear_f16(gpu, orc, m, n, k):
    say("linear f16", m, n, k)
    rng = np.random.default_rng(m * n + k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = (rng.standard_normal(n) * 0.02).astype(np.float32)
    y = gpu.op_linear(w.view(np.uint16), 1, n, k, x, b)
    w32 = w.astype(np.float32)
    ref = orc.linear(x, w32, b)
    exact = x.astype(np.float64) @ w32.T.astype(np.float64) + b
    bound = 2 * (k + 1) * 2.0 ** -24 * (np.abs(x) @ np.abs(w32.T) + np.abs(b))
    assert np.all(np.abs(y - exact) <= bound + 1e-30)
    assert np.abs(y - ref).max() <= 2 * bound.max()


@pytest.mark.parametrize("m,n,k", [(1, 1024, 1024), (1, 64, 4096), (3, 33, 512)])
def test_linear_q8_0(gpu, orc, m, n, k):
    say("linear q8_0", m, n, k)
    rng = np.random.default_rng(7 + k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    raw = synth.quantize_q8_0(w)
    wd = orc.dequant_q8_0(raw, n * k).reshape(n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = gpu.op_linear(raw, 8, n, k, x, None)
    exact = x.astype(np.float64) @ wd.T.astype(np.float64)
    bound = 2 * (k + 1) * 2.0 ** -24 * (np.abs(x) @ np.abs(wd.T))
    assert np.all(np.abs(y - exact) <= bound + 1e-30)


@pytest.mark.parametrize("L", [1, 5, 127, 128, 129, 300, 448, 1500])
def test_attention(gpu, orc, L):
    say("attention kv_len", L)
    rng = np.random.default_rng(L)
    H = 3
    q = rng.standard_normal((H, 64)).astype(np.float32)
    k = rng.standard_normal((H, L, 64)).astype(np.float16)
    v = rng.standard_normal((H, L, 64)).astype(np.float16)
    out = gpu.op_attention(q, k, v)
    for h in range(H):
        ref = orc.attention_head(q[h], k[h].astype(np.float32), v[h].astype(np.float32), 0.125)
        np.testing.assert_allclose(out[h], ref, atol=3e-5, rtol=1e-4)


def test_select(gpu):
    say("select")
    rng = np.random.default_rng(11)
    V = 51864
    lg = rng.standard_normal((3, V)).astype(np.float32)
    lg[0, [10, 20000, 51863]] = 9.0  # tie: first index wins
    lg[1, :] = -np.inf
    lg[1, [7, 3, 9]] = [1.0, 1.0, 0.5]
    mask = np.zeros((3, (V + 31) // 32), np.uint32)
    mask[2, 0] = 0xFFFFFFFF  # suppress ids 0..31
    top = int(np.argmax(lg[2, 32:])) + 32
    lg[2, 5] = 50.0  # masked, must not win
    res = gpu.op_select(lg, k=6, mask=mask)
    assert res[0].argmax == 10 and res[0].topk_ids[:3] == [10, 20000, 51863]
    assert res[1].argmax == 3 and res[1].topk_ids[:3] == [3, 7, 9]
    assert res[1].topk_logits[3] == -np.inf and res[1].topk_ids[3] == 0
    assert res[2].argmax == top
    for r in range(3):
        row = lg[r].astype(np.float64)
        if r == 2:
            row = row.copy()
            row[:32] = -np.inf
        m = row.max()
        lse = m + np.log(np.exp(row - m).sum())
        assert res[r].logsumexp == pytest.approx(lse, abs=2e-5)
        order = sorted(range(V), key=lambda i: (-row[i], i))[:6]
        fin = [i for i in order if np.isfinite(row[i])]
        assert res[r].topk_ids[: len(fin)] == fin


def _oracle_sample(orc, row, temperature, rng_state, history, eot, ts_begin, suppress):
    """The oracle's sampling step of a decode at T > 0 after the first step: the rules, sample with the
    first draw after rng_state, the log-probability of the decode loop (over the rewritten row), and
    the draw's distance from the nearest cumulative-weight edge relative to the total."""
    r = orc.apply_suppress(row, suppress)
    r = orc.ngram_block(orc.ngram_block(r, history, 3), history, 4)
    if ts_begin > 0:
        r = orc.timestamp_rules(r, history, ts_begin, eot, first_step=False)
    u = orc.rng_uniform(rng_state, 1)[0]
    k, w = orc.sample_u(r, temperature, u)
    lp = orc.log_softmax_at(w, k)
    cum = np.cumsum(w.astype(np.float64))
    total = float(np.exp(((r - r.max()) / np.float32(temperature)).astype(np.float64)).sum())
    rr = u * total
    edge = float(np.min(np.abs(cum - rr))) / total
    return k, lp, edge


@pytest.mark.parametrize("V,temperature", [(51864, 0.2), (51864, 0.6), (51865, 1.0), (600, 0.4)])
def test_sample_matches_oracle(gpu, orc, V, temperature):
    """The device sampling step (w4h_op_sample, the kernel the T > 0 decode runs after each step)
    against the oracle's rules + sample + logSoftmax (main/nn/WhisperDecoder.java:176-195, 576-598,
    614-626) on the same row and draw: the same token wherever the draw lies further than 1e-9
    (relative) from a cumulative-weight edge, and the log-probability within 1e-9."""
    rng = np.random.default_rng(V + int(temperature * 10))
    eot, tsb = (V - 50, V - 40) if V > 1000 else (V - 1, -1)
    cases = [
        ([], [], -1),
        ([5, 6, 7, 5, 6], [1, 2, 3], -1),                       # 3-gram repeat: 7 is blocked
        ([9, 8, 7, 6, 9, 8, 7], [], -1),                         # 4-gram repeat: 6 is blocked
        ([11, 12, 13, 14], list(range(20, 60)), tsb),            # text after text: timestamp floor
        ([11, tsb + 3 if tsb > 0 else 3], [], tsb),              # single timestamp after text
        ([11, tsb + 2 if tsb > 0 else 2, tsb + 5 if tsb > 0 else 5], [], tsb),  # timestamp pair
    ]
    checked = 0
    for ci, (hist, sup, ts) in enumerate(cases):
        for rep in range(3):
            row = (rng.standard_normal(V) * 0.5).astype(np.float32)
            if rep == 2:
                row[rng.integers(0, V, 20)] = 4.0  # a few dominant ids
            state = int(rng.integers(0, 2**63))
            mask = gpu.make_mask(1, V, [sup])[0] if sup else None
            tok, lp = gpu.op_sample(row, temperature, state, hist, eot=eot, timestamp_begin=ts, suppress_mask=mask)
            k, lp_o, edge = _oracle_sample(orc, row, temperature, state, hist, eot, ts, sup)
            if edge > 1e-9:
                assert tok == k, f"case {ci}.{rep}: device {tok}, oracle {k} (edge {edge:.2e})"
                assert abs(lp - lp_o) <= 1e-9, f"case {ci}.{rep}: logprob {lp} vs {lp_o}"
                checked += 1
    say(f"sample V={V} T={temperature}: {checked}/{3 * len(cases)} draws compared (the rest lie on an edge)")
    assert checked >= 3 * len(cases) - 2


def test_sample_edge_cases(gpu, orc):
    """Every id but one suppressed: that id is drawn whatever the draw; a row of equal logits draws
    the id the uniform draw falls on (u * V, by the cumulative sum)."""
    V = 1000
    row = np.zeros(V, np.float32)
    mask = gpu.make_mask(1, V, [[i for i in range(V) if i != 617]])[0]
    for state in (1, 99, 2**40 + 3):
        tok, lp = gpu.op_sample(row, 0.7, state, [], eot=V - 1, suppress_mask=mask)
        assert tok == 617
        k, lp_o, _ = _oracle_sample(orc, row, 0.7, state, [], V - 1, -1, [i for i in range(V) if i != 617])
        assert k == 617 and abs(lp - lp_o) <= 1e-9
    for state in (5, 77):
        # every weight is exactly 1, so the cumulative weight of id i is i + 1 and r = u * V
        u = orc.rng_uniform(state, 1)[0]
        tok, lp = gpu.op_sample(row, 1.0, state, [], eot=V - 1)
        assert tok == max(0, math.ceil(u * V) - 1)
        assert abs(lp - (0.0 - math.log(V))) <= 1e-12  # logSoftmax over V weights equal to 1
