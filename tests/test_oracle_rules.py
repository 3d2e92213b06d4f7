"""Pins the oracle's decode rules and drivers (main/nn/WhisperDecoder.java:119-626) with hand-derived
expectations: token histories whose suppressed-id sets are worked out by hand from the reference's
loops, tiny logit tables whose beam-search outcome follows from ordering alone, a needsFallback truth
table, fixed sampling draws, and the published SplitMix64 test vectors of the seeded RNG that stands
in for the reference's unseeded Math.random.  Each expectation is written as a literal, with the
derivation beside it; none is computed by re-running the oracle's own formula.
"""

import math

import numpy as np
import pytest

NEG = -np.inf


def blocked(row):
    return sorted(int(i) for i in np.where(np.isneginf(row))[0])


# ---- applyNgramBlock (:543-564), n = 3 and n = 4 ----------------------------------------------

@pytest.mark.parametrize("gen,n,expect", [
    # suffix (5,7) occurred at i=0 and was followed by 9; windows (7,9),(9,5) do not match
    ([5, 7, 9, 5, 7], 3, [9]),
    # suffix (9,5,7): windows (5,7,9),(7,9,5) do not match
    ([5, 7, 9, 5, 7], 4, []),
    # suffix (1,2) at i=0 and i=3, both followed by 3
    ([1, 2, 3, 1, 2, 3, 1, 2], 3, [3]),
    # suffix (3,1,2) at i=2, followed by g[5]=3
    ([1, 2, 3, 1, 2, 3, 1, 2], 4, [3]),
    # overlapping windows: (4,4) at i=0 -> blocks g[2]=4; the suffix is never compared with itself
    ([4, 4, 4], 3, [4]),
    # genCount 3 = n-1: the loop bound i <= genCount-n is -1, nothing to compare
    ([4, 4, 4], 4, []),
    ([4, 4, 4, 4], 4, [4]),
    # genCount < n-1: nothing
    ([3], 3, []),
    # genCount == n-1 == 2: i <= -1, nothing
    ([3, 3], 3, []),
    # the window starting at the last possible index i = genCount-n: (6,8) at i=2 -> g[4]=2
    ([0, 1, 6, 8, 2, 6, 8], 3, [2]),
    # two different earlier continuations of the same suffix are both blocked
    ([7, 8, 1, 7, 8, 2, 7, 8], 3, [1, 2]),
    # a continuation id outside the vocabulary (900 >= 800) is skipped
    ([1, 2, 900, 1, 2], 3, []),
])
def test_ngram_block(orc, gen, n, expect):
    row = np.zeros(800, np.float32)
    assert blocked(orc.ngram_block(row, gen, n)) == expect


# ---- applyTimestampRules (:484-541) with ts_begin 50, eot 40, 120 tokens ------------------------

TSB, EOT, NV = 50, 40, 120


def allowed(row):
    return [int(i) for i in np.where(~np.isneginf(row))[0]]


def test_timestamp_first_step(orc):
    # first step: <|notimestamps|> (49) and every id below ts_begin go, and ids after ts_begin+50 = 100
    r = orc.timestamp_rules(np.zeros(NV, np.float32), [], TSB, EOT, first_step=True)
    assert allowed(r) == list(range(50, 101))


def test_timestamp_empty_history(orc):
    # not the first step but nothing generated: only <|notimestamps|> is suppressed
    r = orc.timestamp_rules(np.zeros(NV, np.float32), [], TSB, EOT)
    assert blocked(r) == [49]


def test_timestamp_pair(orc):
    # last two generated are timestamps: every timestamp goes; lastTs = 60 adds nothing new
    r = orc.timestamp_rules(np.zeros(NV, np.float32), [55, 60], TSB, EOT)
    assert allowed(r) == list(range(0, 49))


def test_timestamp_single_after_text(orc):
    # single timestamp 62 after text: text ids 0..eot-1 go; timestamps up to lastTs+1 = 63 go
    r = orc.timestamp_rules(np.zeros(NV, np.float32), [55, 7, 8, 62], TSB, EOT)
    assert allowed(r) == list(range(40, 49)) + list(range(63, 120))


def test_timestamp_monotonic_after_text(orc):
    # last token is text: no pair rule; timestamps below the last one (55) go
    r = orc.timestamp_rules(np.zeros(NV, np.float32), [55, 7, 8], TSB, EOT)
    assert blocked(r) == [49] + list(range(50, 55))


def test_timestamp_single_generated(orc):
    # one generated timestamp: penultimateWasTs is true when genCount < 2 -> all timestamps go
    r = orc.timestamp_rules(np.zeros(NV, np.float32), [57], TSB, EOT)
    assert allowed(r) == list(range(0, 49))


def test_suppress_blank_and_list(orc):
    # suppressBlank: eot and id 220 (when the vocabulary has it); applySuppress skips ids out of range
    assert blocked(orc.suppress_blank(np.zeros(300, np.float32), 250)) == [220, 250]
    assert blocked(orc.suppress_blank(np.zeros(100, np.float32), 50)) == [50]
    assert blocked(orc.apply_suppress(np.zeros(10, np.float32), [3, -1, 10, 7, 3])) == [3, 7]


# ---- needsFallback (:435-440) truth table ------------------------------------------------------

@pytest.mark.parametrize("cr,avg,nsp,expect", [
    (2.5, -0.5, 0.1, True),    # compressed too well, speech present
    (2.5, -1.5, 0.7, False),   # compressed too well but no speech and low confidence: accept
    (2.5, -0.5, 0.7, True),    # no speech but confident: the exception needs both
    (2.4, -0.5, 0.1, False),   # 2.4 is not > 2.4, confident
    (2.0, -1.5, 0.1, True),    # low confidence with speech
    (2.0, -1.5, 0.7, False),   # low confidence but no speech
    (2.0, -1.0, 0.1, False),   # -1.0 is not < -1.0
    (2.0, -1.0001, 0.6, True),  # 0.6 is not > 0.6
])
def test_needs_fallback(orc, cr, avg, nsp, expect):
    assert orc.needs_fallback(cr, avg, nsp) is expect


# ---- decodeWithFallback's loop (:119-149) over canned per-temperature results ---------------------

def R(cr, avg, nsp=0.1):
    return {"compression_ratio": cr, "avg_logprob": avg, "no_speech_prob": nsp}


@pytest.mark.parametrize("results,pick,used", [
    # t=0 passes: returned at once
    ([R(1.5, -0.3)] + [R(1.5, -0.2)] * 5, 0, 1),
    # t=0 over-compressed, t=0.2 passes
    ([R(2.6, -0.5), R(1.8, -0.6)] + [R(1.5, -0.2)] * 4, 1, 2),
    # t=0 fails on avg only (ratio <= 2.4): the loop stops after t=0 and returns it
    ([R(1.5, -1.5)] + [R(1.5, -0.2)] * 5, 0, 1),
    # all over-compressed; t=0.4's avg -1.3 < best -0.2 - 1: stop after three decodes, best is t=0
    ([R(3.0, -0.2), R(3.0, -0.5), R(3.0, -1.3), R(1.5, -0.1), R(1.5, -0.1), R(1.5, -0.1)], 0, 3),
    # every temperature fails and stays within 1.0 of the best: all six run, the best avg wins (t=0.2)
    ([R(3.0, -0.9), R(3.0, -0.3), R(3.0, -0.5), R(3.0, -0.6), R(3.0, -0.7), R(3.0, -0.8)], 1, 6),
])
def test_fallback_choice(orc, results, pick, used):
    assert orc.fallback_pick(results) == (pick, used)


# ---- sample (:576-598) with a fixed draw -----------------------------------------------------------

def test_sample_fixed_draws(orc):
    lg = np.log(np.array([1, 2, 3, 4], np.float64)).astype(np.float32)
    # T = 1: weights exp(l - max) = 1/4, 2/4, 3/4, 1 (sum 2.5); r = u * 2.5
    assert orc.sample_u(lg, 1.0, 0.0)[0] == 0      # r = 0: the first cumulative weight already >= 0
    assert orc.sample_u(lg, 1.0, 0.29)[0] == 1     # r = 0.725: 0.25 < r <= 0.75
    assert orc.sample_u(lg, 1.0, 0.5)[0] == 2      # r = 1.25: 0.75 < r <= 1.5
    assert orc.sample_u(lg, 1.0, 0.999)[0] == 3    # r = 2.4975: 1.5 < r <= 2.5
    # T = 0.5 squares the weights: 1/16, 4/16, 9/16, 1 (sum 1.875)
    assert orc.sample_u(lg, 0.5, 0.4)[0] == 2      # r = 0.75: 0.3125 < r <= 0.875
    assert orc.sample_u(lg, 0.5, 0.5)[0] == 3      # r = 0.9375 > 0.875
    # the row is overwritten with the unnormalised weights, as the reference does
    _, w = orc.sample_u(lg, 1.0, 0.5)
    np.testing.assert_allclose(w, [0.25, 0.5, 0.75, 1.0], rtol=1e-6)
    # a suppressed (-inf) id has weight 0 and is never drawn
    assert orc.sample_u(np.array([0, NEG, 0], np.float32), 1.0, 0.6)[0] == 2


def test_splitmix64_published_vectors(orc):
    # Vigna's splitmix64 from seed 1234567 (the published first five outputs)
    assert orc.splitmix64(1234567, 5) == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                                          4593380528125082431, 16408922859458223821]
    # doubles from the top 53 bits: seed 987654321, 100000 draws of floor(5u) (published counts)
    counts = np.bincount([int(u * 5) for u in orc.rng_uniform(987654321, 100000)], minlength=5)
    assert counts.tolist() == [20027, 19892, 20073, 19978, 20030]


# ---- the greedy driver (:161-204) on a logit table ---------------------------------------------------

def table(V, entries):
    r = np.full(V, NEG, np.float32)
    for k, v in entries.items():
        r[k] = v
    return r


def test_greedy_driver_composition(orc):
    V, eot, nsp = 8, 7, 6
    rows = {
        # step 0: eot (7) holds the maximum but suppressBlank removes it; 3 wins over 2
        (): table(V, {7: 5.0, 3: 1.0, 2: 0.0}),
        # step 1: eot wins; its log-prob 2 - ln(e^2 + 1) enters the sum, but not the token count
        (3,): table(V, {7: 2.0, 4: 0.0}),
    }
    src = orc.TableSource(V, lambda h: rows[h], first_row=table(V, {i: 0.0 for i in range(V)} | {nsp: math.log(2)}))
    r = orc.greedy_drive(src, eot, max_tokens=10, no_speech=nsp)
    assert r["tokens"] == [3]
    lp0 = 1.0 - math.log(math.e + 1.0)
    lp1 = 2.0 - math.log(math.e ** 2 + 1.0)
    assert r["avg_logprob"] == pytest.approx(lp0 + lp1, abs=1e-6)
    # no-speech probability: softmax of the prompt's FIRST row at id 6 = 2 / (7 + 2)
    assert r["no_speech_prob"] == pytest.approx(2.0 / 9.0, abs=1e-6)


def test_greedy_driver_rules_order(orc):
    V, eot = 12, 11
    # after a 5 the model prefers 6, otherwise 5; 9 and 10 trail
    pref = table(V, {5: 3.0, 6: 2.0, 9: 1.0, 10: 0.0})

    def rows(h):
        if h and h[-1] == 5:
            return table(V, {6: 3.0, 5: 2.0, 9: 1.0, 10: 0.0})
        return pref

    src = orc.TableSource(V, rows)
    r = orc.greedy_drive(src, eot, max_tokens=6)
    # 5; 6; 5 (no window before genCount 3); 6 (suffix (6,5) never seen);
    # after 5 6 5 6 the suffix (5,6) occurred at 0 followed by 5 -> 5 blocked, 6 taken;
    # after 5 6 5 6 6 neither (6,6) nor (5,6,6) occurred -> 5.  max_tokens = 6 ends it.
    assert r["tokens"] == [5, 6, 5, 6, 6, 5]


# ---- the beam driver (:214-394) on logit tables --------------------------------------------------------

def test_beam_stable_ties_and_finished_cap(orc):
    V, eot, beam = 8, 7, 2
    # step 0: eot suppressed; 0 and 1 tie -> beams [0], [1] with equal log-probs
    # step 1: both beams see 2 and 3 tied; all four candidates score exactly the same, so the stable
    #   sort keeps beam 0's (2, then 3): new beams [0,2] and [0,3]; beam 1's line is dropped
    # step 2: [0,2] -> eot 2, 4 0 ; [0,3] -> 5 0, eot 1.  Scores relative to s: eot via [0,2]
    #   -0.127, eot via [0,3] -0.313, 5 -1.313, 4 -2.127: two finished -> the cap (beam) ends the search
    rows = {
        (): table(V, {0: 0.0, 1: 0.0, 2: -9.0, 3: -9.0, 4: -9.0, 5: -9.0, 6: -9.0, 7: 5.0}),
        (0,): table(V, {2: 1.0, 3: 1.0}),
        (1,): table(V, {2: 1.0, 3: 1.0}),
        (0, 2): table(V, {7: 2.0, 4: 0.0}),
        (0, 3): table(V, {5: 0.0, 7: 1.0}),
    }
    src = orc.TableSource(V, lambda h: rows[h])
    r = orc.beam_drive(src, eot, max_tokens=10, beam=beam)
    assert r["tokens"] == [0, 2]
    s = -math.log(2 + 5 * math.exp(-9.0)) - math.log(2.0)
    assert r["avg_logprob"] == pytest.approx((s + 2.0 - math.log(math.e ** 2 + 1)) / 2, abs=1e-5)
    # hypotheses fed at step 2 are the two beam-0 continuations (tie order), never beam 1's
    assert {h for _, h in src.calls} == {(0,), (1,), (0, 2), (0, 3)}


def test_beam_length_normalised_pick(orc):
    V, eot, beam = 8, 7, 2
    # step 0: [0] (lp a0 = -ln(1 + e^-1)) and [1] (a1 = a0 - 1)
    # step 1: [0] -> eot first: finished F1 = [0] (score a0 - 0.5046, length 1); then [0,2]
    #   (a0 - 1.0046) and [1,4] (a1 - 0.6480) become the beams
    # step 2: [0,2] -> eot: F2 = [0,2] (score a0 - 1.0046 - 0.1269 = -1.4448, length 2) reaches the
    #   cap.  Totals favour F1 (-0.8179 > -1.4448) but per token F2 wins (-0.7224 > -0.8179)
    rows = {
        (): table(V, {0: 0.0, 1: -1.0}),
        (0,): table(V, {7: 0.0, 2: -0.5, 3: -3.0}),
        (1,): table(V, {4: 0.0, 5: -0.1}),
        (0, 2): table(V, {7: 0.0, 6: -2.0}),
        (1, 4): table(V, {3: 0.0}),
    }
    src = orc.TableSource(V, lambda h: rows[h])
    r = orc.beam_drive(src, eot, max_tokens=10, beam=beam)
    assert r["tokens"] == [0, 2]
    a0 = -math.log(1 + math.exp(-1.0))
    f2 = a0 + (-0.5 - math.log(1 + math.exp(-0.5) + math.exp(-3.0))) + (-math.log(1 + math.exp(-2.0)))
    assert r["avg_logprob"] == pytest.approx(f2 / 2, abs=1e-5)


def test_beam_unfinished_fill_at_max_tokens(orc):
    V, eot, beam = 8, 7, 2
    # no eot ever: after max_tokens - 1 = 2 search steps the live beams fill the finished list in
    # beam order and the best per-token score wins.
    # step 0: [0] (a0 = -ln(1 + e^-1)), [1] (a1 = a0 - 1)
    # step 1: [0] -> 2 (0), 3 (-2); [1] -> 4 (0), 5 (-0.5)
    #   scores: [0,2] a0 - ln(1+e^-2) = -0.4402, [1,4] a1 - ln(1+e^-.5) = -1.7873, [1,5] -2.2873,
    #   [0,3] -2.4402 -> beams [0,2], [1,4]
    # step 2: [0,2] -> 6 (0) only: [0,2,6] -0.4402; [1,4] -> 3 (0) only: [1,4,3] -1.7873
    #   (the (beam+1)-th candidates of each beam are id 0 at -inf)
    rows = {
        (): table(V, {0: 0.0, 1: -1.0}),
        (0,): table(V, {2: 0.0, 3: -2.0}),
        (1,): table(V, {4: 0.0, 5: -0.5}),
        (0, 2): table(V, {6: 0.0}),
        (1, 4): table(V, {3: 0.0}),
    }
    src = orc.TableSource(V, lambda h: rows[h])
    r = orc.beam_drive(src, eot, max_tokens=3, beam=beam)
    assert r["tokens"] == [0, 2, 6]
    a0 = -math.log(1 + math.exp(-1.0))
    assert r["avg_logprob"] == pytest.approx((a0 - math.log(1 + math.exp(-2.0))) / 3, abs=1e-5)


# ---- logSoftmax (:614-626) of one entry, as the sampled decode loop takes it --------------------

def test_log_softmax_at_hand_values(orc):
    # (3 - 3) - log(e^-2 + e^-1 + e^0) = -log(1.5032147244) = -0.40760596444
    assert orc.log_softmax_at([1.0, 2.0, 3.0], 2) == pytest.approx(-0.40760596444, abs=1e-10)
    # index 0 of the same row: (1 - 3) - log(1.5032147244) = -2.40760596444
    assert orc.log_softmax_at([1.0, 2.0, 3.0], 0) == pytest.approx(-2.40760596444, abs=1e-10)
    # -inf entries add exp(-inf) = 0: two equal finite entries give log(1/2)
    assert orc.log_softmax_at([NEG, 0.5, 0.5, NEG], 1) == pytest.approx(-math.log(2.0), abs=1e-15)
    # after sample rewrote a row into weights (max weight 1, a suppressed id weight 0): the decode
    # loop's logSoftmax sees weights [1, 0, 1]: (1 - 1) - log(1 + e^-1 + 1) = -log(2.3678794412)
    assert orc.log_softmax_at([1.0, 0.0, 1.0], 0) == pytest.approx(-0.86199480406, abs=1e-10)
