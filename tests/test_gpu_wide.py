"""Decoder-step parity for wide models (d > 512): the step kernels that keep three 16-byte chunk
rounds per lane in registers (d <= 768) and stream the rest of longer rows (d = 1024), with one row
and with several rows (beam-style rows sharing one encoder output, and independent streams).

Contract: per-step logits within max-abs 1e-2 of the oracle (fp32 activations, f16 KV declared),
argmax bit-exact wherever the oracle's top-2 margin exceeds that tolerance.
"""

import numpy as np
import pytest

from whisper4j_amd import synth

pytestmark = pytest.mark.gpu
TOL = 1e-2


def say(*a):
    print("[gpu-wide]", *a, flush=True)


def forced_rows(gpu, dims, T, xas, prompt, forced, n_rows, n_enc):
    m = gpu.Model.from_tensors(dims, T)
    s = m.session(n_rows=n_rows, n_encoders=n_enc)
    for e in range(n_enc):
        s.set_encoder(xas[e], enc=e)
    out = []
    for i, tok in enumerate(list(prompt) + list(forced)):
        res, lg = s.step([tok] * n_rows, want_logits=True, topk=2)
        if i >= len(prompt) - 1:
            out.append((res, lg))
    s.close()
    m.close()
    return out


@pytest.mark.parametrize("d,heads,n_rows,n_enc,wtype", [(768, 12, 1, 1, "f16"), (768, 12, 3, 1, "f16"),
                                                        (1024, 16, 1, 1, "f16"), (1024, 16, 2, 2, "f16"),
                                                        (1024, 16, 1, 1, "q8_0"), (1280, 20, 1, 1, "f16"),
                                                        (1280, 20, 4, 4, "f16")])
def test_wide_forced(gpu, orc, d, heads, n_rows, n_enc, wtype):
    dims = synth.Dims(n_vocab=1200, n_text_ctx=48, n_text_state=d, n_text_head=heads, n_text_layer=2, n_audio_ctx=80)
    say(f"d={d} heads={heads} rows={n_rows} encoders={n_enc} {wtype}")
    T = synth.make_decoder(dims, seed=31, wtype=wtype, ln_random=True)
    xas = [synth.encoder_output(dims, 31, stream=e) for e in range(n_enc)]
    prompt, forced = [1, 2, 3], synth.forced_tokens(12, 31, high=dims.n_vocab - 1)
    om = orc.Model(dims, T)
    refs = [om.forced(xas[e], prompt, forced, want_logits=True) for e in range(n_enc)]
    rows = forced_rows(gpu, dims, T, xas, prompt, forced, n_rows, n_enc)
    worst, agree, covered = 0.0, 0, 0
    for i, (res, lg) in enumerate(rows):
        for r in range(n_rows):
            ref = refs[r if n_enc > 1 else 0]
            worst = max(worst, float(np.abs(lg[r] - ref["logits"][i]).max()))
            if ref["max"][i] - ref["second"][i] > TOL:
                covered += 1
                agree += int(res[r].argmax == ref["argmax"][i])
    say("max-abs", worst, "argmax agree", agree, "/", covered)
    assert worst <= TOL
    assert agree == covered and covered > 0
