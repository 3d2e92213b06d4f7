"""Benchmark: greedy batch-1 decode tokens/s of a Whisper base.en-shaped text decoder on one MI355X.

Workload (the configuration the headline metric is quoted on): d_model 512, 6 layers, 8 heads,
vocab 51864, f16 weights N(0, 0.02), LayerNorm gamma 1 / beta 0, one fp32 [1500, 512] N(0, 1)
encoder output, prompt [50257, 50258, 50359, 50363], then 444 teacher-forced single-token steps
(uniform ids in [0, 50256]) to the full 448-token context.

A bench "step" is one such 444-token decode sweep over device-resident weights, cross-attention
K/V and a self-KV cache holding the prefilled 4-token prompt; each sweep rewinds the KV to the
prompt.  Prefill and the cross-K/V projection are outside the timed region and reported under
"setup" (wall clock, encoder output already in device memory).  Every token step is
a real single-token decoder step (the next token could be the previous argmax; the teacher-forced
id is read from device memory instead).  The whole sweep is one launch of the persistent step
kernel, timed with HIP events on the session stream.

Prints ONE JSON line (see the keys below); ``--gpus N`` with N > 1 exits: the decoder runs on one GPU.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "decode tokens/s (greedy b=1 & beam 5) + % of HBM roofline, 1 MI355X"
N_STEPS = 444
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "k_step_base.en_traffic.txt")


def algorithmic_bytes_per_step(dims, kv_len, rows=1, encoders=1, w_b=2.0, kv_b=2.0):
    """Bytes a decoder step must move: layer weights once, tied logits once, cross K/V of every
    encoder, the self-KV read plus the appended row, biases, LayerNorm parameters, embedding rows."""
    L, d, V, A = dims.n_text_layer, dims.n_text_state, dims.n_vocab, dims.n_audio_ctx
    b = L * 14 * d * d * w_b + V * d * w_b
    b += L * 2 * A * d * kv_b * encoders
    b += rows * L * 2 * d * kv_b * (kv_len + 1)
    b += L * 10 * d * 4 + (3 * L + 1) * 2 * d * 4 + rows * (d * w_b + d * 4)
    return b


def read_traffic():
    if not os.path.exists(TRAFFIC_FILE):
        return None
    for line in open(TRAFFIC_FILE):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def cpu_host():
    """The host CPU the baselines run on: model name, logical CPUs, and the one core they are pinned to."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    allowed = sorted(os.sched_getaffinity(0))
    return {"cpu_model": model, "nproc": os.cpu_count(), "cpus_allowed": len(allowed), "pinned_core": allowed[-1]}


class _Pinned:
    """Runs the enclosed CPU work on one core (as `taskset -c <core>`), restoring the affinity after."""

    def __init__(self, core):
        self.core = core

    def __enter__(self):
        self.old = os.sched_getaffinity(0)
        os.sched_setaffinity(0, {self.core})

    def __exit__(self, *exc):
        os.sched_setaffinity(0, self.old)


def cpu_baseline(dims, T, xa, prompt, forced, min_seconds, max_sweeps, core):
    """The oracle (single-threaded C restatement of the reference's Linux decode path) on a bounded
    sample of the same workload, pinned to one core: whole 444-step teacher-forced sweeps, each after
    an untimed 4-token prefill, repeated until min_seconds of timed CPU work (at most max_sweeps).
    Returns the rate and the records of the last sweep (argmax, max, second, logsumexp per step)."""
    from oracle import oracle as orc

    with _Pinned(core):
        m = orc.Model(dims, T)
        dt, sweeps, rec = 0.0, 0, None
        while sweeps < max_sweeps and (sweeps == 0 or dt < min_seconds):
            c = m.new_cache()
            m.forward(prompt, xa, c)
            t0 = time.perf_counter()
            for i in range(N_STEPS):
                m.forward([int(forced[i])], xa, c)
            dt += time.perf_counter() - t0
            c.close()
            sweeps += 1
        rec = m.forced(xa, prompt, forced[:N_STEPS])
        m.close()
    return N_STEPS * sweeps / dt, dt, sweeps, rec


def cpu_step_rate(name, wtype, seconds, core, rows=1, bias=False):
    """Oracle single-token forwards per second on one core for another workload, after an untimed
    prompt prefill (which includes the cross-K/V projection); `rows` forwards make one step of that
    workload (the reference's beam search runs one batch-1 forward per hypothesis, independent streams
    one per stream).  Returns (steps per second, forwards timed, seconds timed)."""
    from oracle import oracle as orc
    from whisper4j_amd import synth

    dims = synth.SHAPES[name]
    T = synth.make_decoder(dims, seed=0, wtype=wtype)
    forced = synth.forced_tokens(64, 0)
    with _Pinned(core):
        m = orc.Model(dims, T)
        if bias:
            m.set_logit_bias(synth.logit_bias(dims, 0, synth.BEAM_BIAS_SIGMA, synth.EOT_MULTILINGUAL))
        xa = synth.encoder_output(dims, 0)
        c = m.new_cache()
        m.forward(list(synth.BENCH_PREFIX), xa, c)
        n, dt = 0, 0.0
        while n < len(forced) and (n == 0 or dt < seconds):
            t0 = time.perf_counter()
            m.forward([int(forced[n])], xa, c)
            dt += time.perf_counter() - t0
            n += 1
        c.close()
        m.close()
    return n / dt / rows, n, dt


def copy_calibration(mib):
    """A plain device-to-device copy of `mib` MiB (reads mib, writes mib), run three times so that a
    counter pass over this process sees a kernel of known traffic beside the decoder kernel.  Uses the
    HIP runtime directly (hipMemcpy device-to-device runs the runtime's copy kernel); rocprofv3's
    TCC counter passes abort in processes that have loaded torch, so torch is not used here."""
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so")
    n = ctypes.c_size_t(mib << 20)
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    for ptr in (a, b):
        if hip.hipMalloc(ctypes.byref(ptr), n) != 0:
            raise RuntimeError("hipMalloc failed")
    hip.hipMemset(a, 1, n)
    for _ in range(3):
        if hip.hipMemcpy(b, a, n, 3) != 0:  # hipMemcpyDeviceToDevice
            raise RuntimeError("hipMemcpy failed")
    hip.hipDeviceSynchronize()
    hip.hipFree(a)
    hip.hipFree(b)


def traffic_from(fetch_csv, write_csv, copy_mib, out_path):
    """Reduce two rocprofv3 --pmc counter_collection.csv files (FETCH_SIZE pass, WRITE_SIZE pass; both
    in KiB per dispatch) to HBM bytes per sweep launch of the decoder kernel.  The copy kernel of the
    same process (copy_mib read + copy_mib written) calibrates each counter: factor = known bytes /
    counted bytes."""
    import csv

    def per_kernel(path, counter):
        rows = {}
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] != counter:
                continue
            key = (r["Kernel_Name"], r["Dispatch_Id"])
            rows[key] = rows.get(key, 0.0) + float(r["Counter_Value"])
        return rows

    res = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        rows = per_kernel(path, counter)
        step = [v for (k, _), v in rows.items() if "k_step" in k]
        copy = [v for (k, _), v in rows.items() if "copy" in k.lower() or "elementwise" in k.lower()]
        if not step or not copy:
            raise SystemExit(f"{path}: no decoder or copy dispatch with {counter}")
        counted_copy = max(copy) * 1024.0
        factor = (copy_mib << 20) / counted_copy
        counted_step = max(step) * 1024.0  # the sweep launch is the largest decoder dispatch
        res[counter] = (counted_step, counted_copy, factor)
    fetch = res["FETCH_SIZE"][0] * res["FETCH_SIZE"][2]
    write = res["WRITE_SIZE"][0] * res["WRITE_SIZE"][2]
    with open(out_path, "w") as f:
        for counter, (cs, cc, fac) in res.items():
            f.write(f"{counter}: decoder sweep dispatch {cs:.6e} B counted; copy of {copy_mib} MiB counted "
                    f"{cc:.6e} B -> factor {fac:.4f}\n")
        f.write(f"fetch_bytes_per_launch: {fetch:.6e}\n")
        f.write(f"write_bytes_per_launch: {write:.6e}\n")
        f.write(f"traffic_bytes_per_launch: {fetch + write:.6e}\n")
    print(open(out_path).read())


def measure_setup(sess, dims, xas, n_rows, prompt, repeats=3):
    """Per-utterance set-up outside the timed decode steps, with the encoder outputs already in device
    memory: the cross-attention K/V projection of every layer for every encoder (MFMA GEMMs through
    w4h_session_set_encoder_device, one call and synchronisation per encoder), then the 4-token prompt
    prefill (one run call).  Wall clock, median of `repeats` after an untimed first call; leaves the
    session holding the prefilled prompt."""
    from whisper4j_amd.device import DeviceArray

    dev = [DeviceArray(np.asarray(x, dtype=np.float32)) for x in xas]

    def project():
        for e, x in enumerate(dev):
            sess.set_encoder_device(x.address, enc=e)

    project()
    proj = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        project()
        proj.append(time.perf_counter() - t0)
    first = [prompt[0]] * n_rows
    rest = [[t] * n_rows for t in prompt[1:]]
    pre = []
    for _ in range(repeats + 1):
        sess.reset(0)
        t0 = time.perf_counter()
        sess.run(first, forced=rest, n_steps=len(prompt))
        pre.append(time.perf_counter() - t0)
    for x in dev:
        x.close()
    L, d, A = dims.n_text_layer, dims.n_text_state, dims.n_audio_ctx
    flop = 2 * 2 * L * A * d * d * len(xas)
    p = float(np.median(proj))
    return {"cross_kv_ms": round(p * 1e3, 4), "cross_kv_gflop": round(flop / 1e9, 2),
            "cross_kv_tflop_s": round(flop / p / 1e12, 1), "prefill_ms": round(float(np.median(pre[1:])) * 1e3, 4)}


def measure_forced(w4h, synth, name, wtype, n_steps, repeats, n_rows=1, n_encoders=1, n_sessions=1):
    """Teacher-forced decode of one config: 4-token prefix prefilled untimed, then `n_steps` steps in
    one launch per session and repeat; returns (tokens/s over all rows and sessions, us per step,
    roofline fraction of the mean step, set-up costs of the first session)."""
    dims = synth.SHAPES[name]
    T = synth.make_decoder(dims, seed=0, wtype=wtype)
    model = w4h.Model.from_tensors(dims, T)
    prompt = list(synth.BENCH_PREFIX)
    forced = synth.forced_tokens(n_steps, 0)
    sessions = []
    setup = None
    for q in range(n_sessions):
        sess = model.session(n_rows=n_rows, n_encoders=n_encoders, max_ctx=dims.n_text_ctx)
        xas = [synth.encoder_output(dims, 0, stream=q * n_encoders + e) for e in range(n_encoders)]
        if q == 0:
            setup = measure_setup(sess, dims, xas, n_rows, prompt)
        else:
            for e in range(n_encoders):
                sess.set_encoder(xas[e], enc=e)
            first = [prompt[0]] * n_rows
            rest = [[t] * n_rows for t in prompt[1:]]
            sess.run(first, forced=rest, n_steps=len(prompt))
        sessions.append(sess)
    kv0 = sessions[0].kv_len
    tok0 = [int(forced[0])] * n_rows
    fwd = [[int(t)] * n_rows for t in forced[1:n_steps]]
    for sess in sessions:
        sess.time_run(tok0, fwd, n_steps, 1)  # warm-up
    total_ms = 0.0
    for sess in sessions:
        ms, _ = sess.time_run(tok0, fwd, n_steps, repeats)
        total_ms += float(np.mean(ms))
    for sess in sessions:
        sess.close()
    model.close()
    step_us = total_ms * 1e3 / n_steps
    w_b = 34.0 / 32.0 if wtype == "q8_0" else 2.0
    rows = n_rows * n_sessions
    encs = n_encoders * n_sessions
    byts = sum(algorithmic_bytes_per_step(dims, kv0 + i, rows=rows, encoders=encs, w_b=w_b) for i in range(n_steps))
    frac = byts / (total_ms * 1e-3) / 1e9 / HBM_PEAK_GBS
    return rows * n_steps / (total_ms * 1e-3), step_us, frac, setup


def measure_beam(w4h, synth, name, n_steps, beam):
    """Beam search through the library's beam driver (w4h_decode_beam: the prompt prefill, then for a
    batched session candidate scoring, sorting, finished list, masks and KV reorder on the device in
    32-step launches), with the workload's seeded logit bias N(0, 1) and the end token at -inf, so every
    hypothesis runs all steps.  Returns (steps/s, hypothesis tokens/s, us per step, steps, roofline
    fraction of the mean step: the 5 rows' bytes per step over the measured step time)."""
    from whisper4j_amd.decoder import WhisperDecoder

    dims = synth.SHAPES[name]
    T = synth.make_decoder(dims, seed=0, wtype="f16")
    model = w4h.Model.from_tensors(dims, T)
    dec = WhisperDecoder(model, beam_size=beam)
    dec.set_logit_bias(synth.logit_bias(dims, 0, synth.BEAM_BIAS_SIGMA, synth.EOT_MULTILINGUAL))
    xa = synth.encoder_output(dims, 0)
    eot = synth.EOT_MULTILINGUAL
    prompt = list(synth.BENCH_PREFIX)
    dec.decode_beam(xa, prompt, eot, 16)  # warm-up
    t0 = time.perf_counter()
    r = dec.decode_beam(xa, prompt, eot, n_steps)
    dt = time.perf_counter() - t0
    dec.close()
    model.close()
    steps = len(r.tokens)
    kv0 = len(prompt)
    byts = sum(algorithmic_bytes_per_step(dims, kv0 + i, rows=beam, encoders=1) for i in range(steps))
    frac = byts / dt / 1e9 / HBM_PEAK_GBS
    return steps / dt, beam * steps / dt, dt * 1e6 / steps, steps, frac


def measure_greedy_driver(w4h, synth, name, n_tokens):
    """The library's greedy decode driver (w4h_decode: prompt prefill, then the decode with the
    suppress, n-gram and timestamp rules; EOT suppressed so every token runs), with the rules on the
    device (one launch that ends at the end token) and, for comparison, driven from the host (one
    step call and host round trip per token).  Returns {mode: (tokens/s, us per token)}."""
    from whisper4j_amd.decoder import WhisperDecoder

    dims = synth.SHAPES[name]
    T = synth.make_decoder(dims, seed=0, wtype="f16")
    model = w4h.Model.from_tensors(dims, T)
    xa = synth.encoder_output(dims, 0)
    eot, tsb = 50256, 50363
    prompt = list(synth.BENCH_PREFIX)
    out = {}
    old = os.environ.get("W4H_DEVICE_RULES")
    for mode, env in (("device_rules", "1"), ("host_loop", "0")):
        os.environ["W4H_DEVICE_RULES"] = env
        dec = WhisperDecoder(model, beam_size=1, max_ctx=dims.n_text_ctx)
        dec.decode(xa, prompt, eot, 16, suppress_tokens=[eot], timestamp_begin=tsb)  # warm-up
        t0 = time.perf_counter()
        r = dec.decode(xa, prompt, eot, n_tokens, suppress_tokens=[eot], timestamp_begin=tsb)
        dt = time.perf_counter() - t0
        dec.close()
        out[mode] = (len(r.tokens) / dt, dt * 1e6 / len(r.tokens))
    if old is None:
        os.environ.pop("W4H_DEVICE_RULES", None)
    else:
        os.environ["W4H_DEVICE_RULES"] = old
    model.close()
    return out


def measure_sampled_driver(w4h, synth, name, n_tokens, temperature=0.6, seed=3):
    """The library's decode driver at temperature > 0 (w4h_decode: prompt prefill, then sampled
    tokens with the suppress, n-gram and timestamp rules; EOT suppressed so every token runs), with
    the sampling on the device (a sampling kernel chained after each one-step launch, no host round
    trip per token) and, for comparison, on the host (each logits row fetched and sampled there).
    Returns {mode: (tokens/s, us per token)}."""
    from whisper4j_amd.decoder import WhisperDecoder

    dims = synth.SHAPES[name]
    T = synth.make_decoder(dims, seed=0, wtype="f16")
    model = w4h.Model.from_tensors(dims, T)
    xa = synth.encoder_output(dims, 0)
    eot, tsb = 50256, 50363
    prompt = list(synth.BENCH_PREFIX)
    out = {}
    old = os.environ.get("W4H_DEVICE_SAMPLE")
    for mode, env in (("device_sampling", "1"), ("host_loop", "0")):
        os.environ["W4H_DEVICE_SAMPLE"] = env
        dec = WhisperDecoder(model, beam_size=1, max_ctx=dims.n_text_ctx)
        dec.decode(xa, prompt, eot, 16, suppress_tokens=[eot], temperature=temperature, seed=seed, timestamp_begin=tsb)
        t0 = time.perf_counter()
        r = dec.decode(xa, prompt, eot, n_tokens, suppress_tokens=[eot], temperature=temperature, seed=seed,
                       timestamp_begin=tsb)
        dt = time.perf_counter() - t0
        dec.close()
        out[mode] = (len(r.tokens) / dt, dt * 1e6 / len(r.tokens))
    if old is None:
        os.environ.pop("W4H_DEVICE_SAMPLE", None)
    else:
        os.environ["W4H_DEVICE_SAMPLE"] = old
    model.close()
    return out


def encoder_flops(ed):
    """Algorithmic FLOPs of one encoder forward: conv1 over 2T frames, conv2 over T, per layer the
    q/k/v/out projections and the MLP (24 T d^2) and the attention products (4 T^2 d)."""
    T, d, nm, L = ed.n_audio_ctx, ed.n_audio_state, ed.n_mels, ed.n_audio_layer
    conv = 2 * (2 * T) * d * 3 * nm + 2 * T * d * 3 * d
    gemm = L * 24 * T * d * d
    attn = L * 4 * T * T * d
    return conv + gemm, attn


def measure_encoder(w4h, synth, name, reps=5):
    """WhisperEncoder.forward on the GPU (w4h_encoder_forward_device: mel and output in device memory,
    the call returns when the output is written), seed-0 f16 weights and mel, wall clock per forward
    over `reps` forwards after one warm-up.  MFMA work: two f16 products per GEMM multiply-add
    (activation hi/lo) and three per attention product."""
    from whisper4j_amd.device import DeviceArray

    ed = synth.ENC_SHAPES[name]
    T = synth.make_encoder(ed, seed=0)
    mel = synth.mel_input(ed, 0)
    enc = w4h.Encoder.from_tensors(ed, T)
    with DeviceArray(mel) as dm, DeviceArray(np.zeros((ed.n_audio_ctx, ed.n_audio_state), np.float32)) as dx:
        enc.forward_device(dm.address, dx.address)
        t0 = time.perf_counter()
        for _ in range(reps):
            enc.forward_device(dm.address, dx.address)
        dt = (time.perf_counter() - t0) / reps
    enc.close()
    gf, af = encoder_flops(ed)
    mfma = 2 * gf + 3 * af
    return {"ms": round(dt * 1e3, 3), "gflop": round((gf + af) / 1e9, 1), "tflop_s": round((gf + af) / dt / 1e12, 1),
            "mfma_tflop_s": round(mfma / dt / 1e12, 1), "mfma_frac_of_f16_peak": round(mfma / dt / 2.5e15, 4)}


def other_configs(w4h, synth):
    """Absolute decode rates of the four other workload shapes (one bounded run each)."""
    out = {}
    tps, us, frac, setup = measure_forced(w4h, synth, "tiny.en", "f16", 224, 5)
    out["tiny.en greedy b=1, 224 forced steps"] = {"tokens_per_s": round(tps, 1), "us_per_step": round(us, 2),
                                                   "roofline_frac": round(frac, 4), "setup": setup}
    drv = measure_greedy_driver(w4h, synth, "base.en", 224)
    out["base.en greedy decode driver w4h_decode, 224 tokens (prompt prefill, then suppress + n-gram + timestamp rules; EOT suppressed)"] = {
        "tokens_per_s": round(drv["device_rules"][0], 1), "us_per_token": round(drv["device_rules"][1], 2),
        "rules": "on the device, one launch",
        "host_loop_tokens_per_s": round(drv["host_loop"][0], 1), "host_loop_us_per_token": round(drv["host_loop"][1], 2)}
    smp = measure_sampled_driver(w4h, synth, "base.en", 224)
    out["base.en sampled decode driver w4h_decode at T = 0.6, 224 tokens (prompt prefill, then sampled tokens with suppress + n-gram + timestamp rules; EOT suppressed)"] = {
        "tokens_per_s": round(smp["device_sampling"][0], 1), "us_per_token": round(smp["device_sampling"][1], 2),
        "sampling": "on the device, each token drawn inside the step kernel (one launch per 64 tokens)",
        "host_loop_tokens_per_s": round(smp["host_loop"][0], 1), "host_loop_us_per_token": round(smp["host_loop"][1], 2)}
    sps, hps, us, steps, frac = measure_beam(w4h, synth, "small", 224, 5)
    out["small beam 5, 224 steps (library beam driver w4h_decode_beam: prompt prefill, then the search on the device; seeded logit bias N(0,1), end token at -inf)"] = {
        "steps_per_s": round(sps, 1), "hypothesis_tokens_per_s": round(hps, 1), "us_per_step": round(us, 2),
        "steps": steps, "roofline_frac": round(frac, 4)}
    tps, us, frac, setup = measure_forced(w4h, synth, "small", "f16", 224, 2, n_rows=5, n_encoders=1)
    out["small 5 beam rows on one encoder, 224 forced steps in one run (device step only)"] = {
        "steps_per_s": round(1e6 / us, 1), "hypothesis_tokens_per_s": round(tps, 1), "us_per_step": round(us, 2),
        "roofline_frac": round(frac, 4), "setup": setup}
    tps, us, frac, setup = measure_forced(w4h, synth, "large-v3-turbo", "f16", 224, 2, n_rows=32, n_encoders=32)
    out["large-v3-turbo 32 streams (own encoder each) in lockstep, 224 forced steps (batched MFMA engine)"] = {
        "tokens_per_s": round(tps, 1), "us_per_step": round(us, 2), "roofline_frac": round(frac, 4), "setup": setup}
    tps, us, frac, setup = measure_forced(w4h, synth, "medium", "q8_0", 444, 2)
    out["medium q8_0 greedy b=1, 444 forced steps"] = {"tokens_per_s": round(tps, 1), "us_per_step": round(us, 2),
                                                      "roofline_frac": round(frac, 4), "setup": setup}
    out["audio encoder forward (80/128 mels x 3000 frames -> 1500 frames, f16 weights, MFMA)"] = {
        name: measure_encoder(w4h, synth, name) for name in ("tiny.en", "base.en", "large-v3-turbo")}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10, help="timed 444-token decode sweeps")
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="minimum timed oracle work for the CPU baseline")
    ap.add_argument("--cpu-max-sweeps", type=int, default=8)
    ap.add_argument("--cpu-config-seconds", type=float, default=2.0,
                    help="timed oracle forwards per other workload for its CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the tiny/small/turbo/medium lines")
    ap.add_argument("--only", choices=["turbo", "small-beam-rows", "small-beam", "greedy-driver", "sampled-driver", "medium",
                                       "tiny", "encoder"],
                    help="run only this other workload (one JSON line; for profiling it alone)")
    ap.add_argument("--only-steps", type=int, default=224, help="forced steps of the --only workload")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="also run a plain copy of this many MiB (counter calibration for rocprofv3 --pmc)")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="reduce two --pmc counter CSVs to the traffic file and exit (no GPU work)")
    args = ap.parse_args()
    if args.traffic_from:
        traffic_from(args.traffic_from[0], args.traffic_from[1], args.copy_mib or 256, TRAFFIC_FILE)
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}); the decoder has no multi-GPU path.",
              file=sys.stderr)
        sys.exit(2)

    import whisper4j_amd as w4h
    from whisper4j_amd import synth

    if args.only:
        n = args.only_steps
        if args.only == "greedy-driver":
            drv = measure_greedy_driver(w4h, synth, "base.en", n)
            print(json.dumps({"workload": f"base.en greedy decode driver, {n} tokens",
                              **{k: {"tokens_per_s": round(v[0], 1), "us_per_token": round(v[1], 2)} for k, v in drv.items()}}))
            return
        if args.only == "encoder":
            print(json.dumps({"workload": "audio encoder forward", **{k: measure_encoder(w4h, synth, k)
                                                                       for k in ("tiny.en", "base.en", "large-v3-turbo")}}))
            return
        if args.only == "small-beam":
            sps, hps, us, steps, frac = measure_beam(w4h, synth, "small", n, 5)
            print(json.dumps({"workload": f"small beam 5 through the library beam driver, {n} steps",
                              "steps_per_s": round(sps, 1), "hypothesis_tokens_per_s": round(hps, 1), "us_per_step": round(us, 2),
                              "steps": steps, "roofline_frac": round(frac, 4)}))
            return
        if args.only == "sampled-driver":
            drv = measure_sampled_driver(w4h, synth, "base.en", n)
            print(json.dumps({"workload": f"base.en sampled decode driver (T = 0.6), {n} tokens",
                              **{k: {"tokens_per_s": round(v[0], 1), "us_per_token": round(v[1], 2)} for k, v in drv.items()}}))
            return
        if args.only == "turbo":
            tps, us, frac, setup = measure_forced(w4h, synth, "large-v3-turbo", "f16", n, 2, n_rows=32, n_encoders=32)
            work = f"large-v3-turbo 32 streams (own encoder each) in lockstep, {n} forced steps"
        elif args.only == "medium":
            tps, us, frac, setup = measure_forced(w4h, synth, "medium", "q8_0", n, 2)
            work = f"medium q8_0 greedy b=1, {n} forced steps"
        elif args.only == "tiny":
            tps, us, frac, setup = measure_forced(w4h, synth, "tiny.en", "f16", n, 5)
            work = f"tiny.en greedy b=1, {n} forced steps"
        else:
            tps, us, frac, setup = measure_forced(w4h, synth, "small", "f16", n, 2, n_rows=5, n_encoders=1)
            work = f"small 5 beam rows on one encoder, {n} forced steps"
        if args.copy_mib:
            copy_calibration(args.copy_mib)
        print(json.dumps({"workload": work, "tokens_per_s": round(tps, 1), "us_per_step": round(us, 2),
                          "roofline_frac": round(frac, 4), "setup": setup}))
        return

    dims = synth.SHAPES["base.en"]
    T = synth.make_decoder(dims, seed=0, wtype="f16")
    xa = synth.encoder_output(dims, 0)
    prompt = list(synth.BENCH_PREFIX)
    forced = synth.forced_tokens(N_STEPS, 0)

    model = w4h.Model.from_tensors(dims, T)
    sess = model.session(n_rows=1, max_ctx=dims.n_text_ctx)
    setup = measure_setup(sess, dims, [xa], 1, prompt)  # cross K/V + prefill, outside the timed sweeps
    kv0 = sess.kv_len
    # sweep: forced[i] at position 4 + i for i < 444 (kv_len 4 -> 448)
    tok0 = [int(forced[0])]
    fwd = forced[1:N_STEPS]
    if args.warmup:
        sess.time_run(tok0, fwd, N_STEPS, args.warmup)
    t0 = time.perf_counter()
    ms, outs = sess.time_run(tok0, fwd, N_STEPS, args.steps)
    wall = time.perf_counter() - t0
    sess.close()
    model.close()
    if args.copy_mib:
        copy_calibration(args.copy_mib)

    ms_mean = float(np.mean(ms))
    tok_s = N_STEPS * args.steps / wall
    bytes_launch = sum(algorithmic_bytes_per_step(dims, kv0 + i) for i in range(N_STEPS))
    achieved = bytes_launch / (ms_mean * 1e-3) / 1e9
    traffic = read_traffic()

    configs = None if args.no_configs else other_configs(w4h, synth)

    cpu, parity = None, None
    if not args.no_cpu:
        host = cpu_host()
        core = host["pinned_core"]
        cps, dt, sweeps, rec = cpu_baseline(dims, T, xa, prompt, forced, args.cpu_seconds, args.cpu_max_sweeps, core)
        cpu = {"value": round(cps, 3), "unit": "tokens/s", "cores": 1, "kind": "port",
               "sample": f"the same base.en workload on the oracle: {sweeps} whole {N_STEPS}-step teacher-forced "
                         f"sweeps (positions 4..447, each after an untimed 4-token prefill), one thread pinned to "
                         f"core {core}, {dt:.1f} s timed",
               "host": host}
        # parity of the timed sweep: device record i follows forced[i], the oracle's row i + 1
        am = np.array([o[0].argmax for o in outs])
        mx = np.array([o[0].max_logit for o in outs])
        lse = np.array([o[0].logsumexp for o in outs])
        covered = (rec["max"] - rec["second"])[1:] > 1e-2
        parity = {"tol": 1e-2, "steps": int(len(am)), "margin_coverage": round(float(covered.mean()), 4),
                  "argmax_equal_where_covered": f"{int((am[covered] == rec['argmax'][1:][covered]).sum())}/{int(covered.sum())}",
                  "max_abs_dmax": float(np.abs(mx - rec["max"][1:]).max()),
                  "max_abs_dlogsumexp": float(np.abs(lse - rec["lse"][1:]).max())}
        if not args.no_configs:
            cfg = {}
            for key, name, wtype, rows, unit, note in (
                    ("tiny.en", "tiny.en", "f16", 1, "tokens/s", "greedy b=1"),
                    ("small beam 5", "small", "f16", 5, "beam steps/s",
                     "one beam step = 5 batch-1 forwards (the reference runs one per hypothesis), seeded logit bias"),
                    ("large-v3-turbo 32 streams", "large-v3-turbo", "f16", 1, "tokens/s",
                     "per stream; the 32 streams run one after another on one core at this rate"),
                    ("medium q8_0", "medium", "q8_0", 1, "tokens/s", "greedy b=1, weights dequantized to fp32")):
                rate, n, t = cpu_step_rate(name, wtype, args.cpu_config_seconds, core, rows=rows,
                                           bias=name == "small")
                cfg[key] = {"value": round(rate, 3), "unit": unit, "cores": 1, "kind": "port",
                            "sample": f"{n} single-token forwards on the oracle after an untimed prompt prefill, "
                                      f"{t:.1f} s timed; {note}"}
            cpu["configs"] = cfg

    line = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 weights / fp32 compute / f16 KV",
        "data": "synthetic (seeded random-init weights, N(0,1) encoder output, uniform teacher-forced ids)",
        "config": {"workload": "whisper base.en-shaped decoder, greedy batch 1, 4-token prefix + 444 teacher-forced "
                               "steps to the 448-token context (one step = one 444-token sweep)",
                   "d_model": 512, "layers": 6, "heads": 8, "vocab": 51864, "tokens_per_step": N_STEPS,
                   "kernel_ms_per_step": round(ms_mean, 4),
                   "us_per_token": round(ms_mean * 1e3 / N_STEPS, 3)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "w4h::k_step<1,0> (persistent decoder step, whole sweep per launch)",
                     "algorithmic_bytes_per_launch": int(bytes_launch)},
        "cpu_baseline": cpu,
        "parity": parity,
        "setup": setup,
        "other_configs": configs,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
