"""Writes the oracle's results at the five benchmark workloads as fixtures for the GPU parity tests.

Every workload is the benchmark's own: the full model shape, seed-0 weights and encoder outputs from
whisper4j_amd.synth, the prompt [50257, 50258, 50359, 50363] and the seed-0 teacher-forced ids.  The
oracle (oracle/libwhisper_ref.so, the CPU restatement of the reference decoder) runs each one here,
in the build container, and only its results are kept:

  tiny.en        4-token prompt + 224 forced steps: per-step argmax, max, second-largest and
                 log-sum-exp logits, and full logits rows at steps 0 and 224
  base.en        prompt + 444 forced steps to the 448-token context (as above, rows at 0 and 444),
                 and a free-running greedy decode of 444 tokens with the decode rules (tokens, the
                 top-2 margin of the masked logits at every step, average log-probability)
  small_beam5    beam search, beam 5, 224 tokens, with the seeded logit bias N(0, 1) and the end
                 token at -inf: tokens, average log-probability and the decision gap of every search
                 step (the last hypothesis kept against the first candidate left out; permuted
                 hypotheses of the biased ids tie to ~1e-4 now and then), and the same search cut at
                 4 to 64 tokens and before the first decision gap below 2e-3
  large-v3-turbo 32 streams, each with its own encoder output, 224 forced steps: per-step records
                 of every stream, full rows of stream 0 at steps 0 and 224
  medium_q8_0    q8_0 weights, prompt + 444 forced steps (records, rows at 0 and 444)

Usage (about three minutes on 8 cores):  python tests/golden/make_config_fixtures.py [--only NAME]
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT = os.path.join(HERE, "configs")
sys.path.insert(0, ROOT)

from whisper4j_amd import synth  # noqa: E402

PROMPT = list(synth.BENCH_PREFIX)
FORCED = {
    "tiny.en": dict(shape="tiny.en", wtype="f16", steps=224, rows_at=(0, 224)),
    "base.en": dict(shape="base.en", wtype="f16", steps=444, rows_at=(0, 444), greedy=444, eot=50256),
    "medium_q8_0": dict(shape="medium", wtype="q8_0", steps=444, rows_at=(0, 444)),
}
TURBO = dict(shape="large-v3-turbo", wtype="f16", steps=224, streams=32, rows_at=(0, 224))
BEAM = dict(shape="small", wtype="f16", beam=5, max_tokens=224, sigma=synth.BEAM_BIAS_SIGMA,
            eot=synth.EOT_MULTILINGUAL)


def _oracle():
    from oracle import oracle as orc

    orc.lib()
    return orc


def forced_records(shape, wtype, steps, stream=0, rows_at=()):
    orc = _oracle()
    dims = synth.SHAPES[shape]
    T = synth.make_decoder(dims, seed=0, wtype=wtype)
    xa = synth.encoder_output(dims, 0, stream=stream)
    forced = synth.forced_tokens(steps, 0)
    m = orc.Model(dims, T)
    r = m.forced(xa, PROMPT, forced, want_logits=bool(rows_at))
    m.close()
    out = {k: r[k] for k in ("argmax", "max", "second", "lse")}
    if rows_at:
        out["rows"] = np.stack([r["logits"][i] for i in rows_at])
    return out


def greedy_path(shape, wtype, n_tokens, eot):
    """The oracle's free-running greedy decode (suppressBlank at the first step, n-gram rules) and the
    top-2 margin of the masked logits at each of its steps."""
    orc = _oracle()
    dims = synth.SHAPES[shape]
    T = synth.make_decoder(dims, seed=0, wtype=wtype)
    xa = synth.encoder_output(dims, 0)
    m = orc.Model(dims, T)
    g = m.decode(xa, PROMPT, eot=eot, max_tokens=n_tokens)
    toks = list(g["tokens"])
    feed = toks[:-1] if len(toks) == n_tokens else toks  # rows exist for every decided step
    lg = m.forced(xa, PROMPT, np.array(feed, np.int32), want_logits=True)["logits"]
    m.close()
    margins = []
    for i in range(len(lg)):
        row = lg[i]
        if i == 0:
            row = orc.suppress_blank(row, eot)
        row = orc.ngram_block(orc.ngram_block(row, toks[:i], 3), toks[:i], 4)
        top2 = np.sort(row)[-2:]
        margins.append(float(top2[1] - top2[0]))
    return {"greedy_tokens": np.array(toks, np.int32), "greedy_margin": np.array(margins, np.float32),
            "greedy_avg_logprob": np.float32(g["avg_logprob"])}


BEAM_GATE = 2e-3  # decisions whose gap is above this are compared token for token


def beam_result():
    orc = _oracle()
    dims = synth.SHAPES[BEAM["shape"]]
    T = synth.make_decoder(dims, seed=0, wtype=BEAM["wtype"])
    xa = synth.encoder_output(dims, 0)
    m = orc.Model(dims, T)
    m.set_logit_bias(synth.logit_bias(dims, 0, BEAM["sigma"], BEAM["eot"]))
    kw = dict(eot=BEAM["eot"], beam=BEAM["beam"])
    r, gaps = m.decode_beam_gaps(xa, PROMPT, max_tokens=BEAM["max_tokens"], **kw)
    out = {"beam_tokens": np.array(r["tokens"], np.int32), "beam_avg_logprob": np.float32(r["avg_logprob"]),
           "beam_gaps": gaps}
    # the search cut at length k runs the same first k - 1 steps as the full search
    small = np.where(gaps[1:] <= BEAM_GATE)[0]
    k_safe = int(small[0]) + 1 if small.size else BEAM["max_tokens"]
    cuts = sorted({k for k in (4, 6, 8, 10, 12, 16, 24, 32, 48, 64, k_safe) if 2 <= k <= BEAM["max_tokens"]})
    for k in cuts:
        rk, gk = m.decode_beam_gaps(xa, PROMPT, max_tokens=k, **kw)
        out[f"cut{k}_tokens"] = np.array(rk["tokens"], np.int32)
        out[f"cut{k}_avg_logprob"] = np.float32(rk["avg_logprob"])
        out[f"cut{k}_gaps"] = gk
    out["cuts"] = np.array(cuts, np.int32)
    m.close()
    return out


def _save(name, meta, arrays):
    os.makedirs(OUT, exist_ok=True)
    path = os.path.join(OUT, f"{name}.npz")
    np.savez_compressed(path, meta=np.array(json.dumps(meta)), **arrays)
    print(f"{path}: {os.path.getsize(path) / 1024:.0f} KiB", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--only")
    ap.add_argument("--workers", type=int, default=8)
    args = ap.parse_args()
    want = lambda n: args.only in (None, n)  # noqa: E731
    t0 = time.time()
    with cf.ProcessPoolExecutor(max_workers=args.workers) as ex:
        futs = {}
        for name, c in FORCED.items():
            if want(name):
                futs[ex.submit(forced_records, c["shape"], c["wtype"], c["steps"], 0, c["rows_at"])] = (name, None)
                if "greedy" in c:
                    futs[ex.submit(greedy_path, c["shape"], c["wtype"], c["greedy"], c["eot"])] = (name, "greedy")
        if want("large-v3-turbo"):
            for s in range(TURBO["streams"]):
                futs[ex.submit(forced_records, TURBO["shape"], TURBO["wtype"], TURBO["steps"], s,
                               TURBO["rows_at"] if s == 0 else ())] = ("large-v3-turbo", s)
        if want("small_beam5"):
            futs[ex.submit(beam_result)] = ("small_beam5", None)
        res = {}
        for f in cf.as_completed(futs):
            name, part = futs[f]
            res.setdefault(name, {})[part] = f.result()
            print(f"{name} {part} done at {time.time() - t0:.0f} s", flush=True)
    for name, c in FORCED.items():
        if name in res:
            arrays = dict(res[name][None])
            if "greedy" in res[name]:
                arrays.update(res[name]["greedy"])
            meta = dict(c, prompt=PROMPT, seed=0, rows_at=list(c["rows_at"]))
            _save(name, meta, arrays)
    if "large-v3-turbo" in res:
        parts = res["large-v3-turbo"]
        arrays = {k: np.stack([parts[s][k] for s in range(TURBO["streams"])]) for k in ("argmax", "max", "second", "lse")}
        arrays["rows"] = parts[0]["rows"]
        _save("large-v3-turbo", dict(TURBO, prompt=PROMPT, seed=0, rows_at=list(TURBO["rows_at"])), arrays)
    if "small_beam5" in res:
        _save("small_beam5", dict(BEAM, prompt=PROMPT, seed=0), res["small_beam5"][None])


if __name__ == "__main__":
    main()
