"""The audio encoder on the GPU (w4h_encoder_*, w4h_encoder.hip: MFMA GEMMs with f16 hi/lo operands,
MFMA flash attention, implicit-GEMM convolutions) against the oracle's restatement of
WhisperEncoder.forward (main/nn/WhisperEncoder.java:42-76).

Bar: the encoder output (LayerNorm rows of unit scale) within max |d| 4e-3 and mean |d| 3e-4 of the
oracle; the oracle itself is pinned to a float64 formulation at 2e-3 / 2e-4 (tests/test_oracle_encoder.py).
The two products per weight (activation hi/lo) and three per attention product keep ~22 bits of
each fp32 operand; what remains is float32 summation order and GELU inputs on an f16 rounding edge."""

import os
import tempfile

import numpy as np
import pytest

from whisper4j_amd import synth

pytestmark = pytest.mark.gpu


def say(*a):
    print("[gpu-enc]", *a, flush=True)


def _check(y, ref, tag, max_tol=4e-3, mean_tol=3e-4):
    err = np.abs(y - ref)
    say(f"{tag}: max |d| {err.max():.2e}, mean |d| {err.mean():.2e}")
    assert np.isfinite(y).all()
    assert err.max() <= max_tol
    assert err.mean() <= mean_tol


@pytest.mark.parametrize("wtype,edims", [
    ("f16", synth.EncDims(80, 48, 128, 2, 2)),        # one key block, frames not a multiple of 64
    ("q8_0", synth.EncDims(16, 40, 128, 2, 1)),
    ("f16", synth.EncDims(128, 33, 192, 3, 1)),       # large-v3 mel count, 3 heads
    ("f16", synth.EncDims(80, 150, 256, 4, 2)),       # three key blocks, the last partial
    ("q8_0", synth.EncDims(80, 130, 256, 4, 2)),
    ("f16", synth.EncDims(80, 300, 384, 6, 1)),       # conv1 over 600 frames: five 128-row tiles
])
def test_encoder_matches_oracle(gpu, orc, wtype, edims):
    say(f"encoder {wtype} {edims}")
    T = synth.make_encoder(edims, seed=5, wtype=wtype, ln_random=True, qk_std=0.1)
    mel = synth.mel_input(edims, 5)
    oe = orc.Encoder(edims, T)
    ref = oe.forward(mel)
    oe.close()
    with gpu.Encoder.from_tensors(edims, T) as enc:
        y = enc.forward(mel)
        y2 = enc.forward(mel)
    _check(y, ref, f"{wtype} T={edims.n_audio_ctx} d={edims.n_audio_state}")
    np.testing.assert_array_equal(y, y2)  # deterministic across calls


def test_encoder_ggml_file_matches_tensors(gpu):
    """A GGML file with encoder hparams and tensors (synth.write_ggml) loads through
    w4h_encoder_load_ggml (model/GgmlLoader.java:95-216 layout) to the same output, bit for bit, as
    w4h_encoder_create from the same tensors."""
    edims = synth.EncDims(80, 64, 128, 2, 2)
    dims = synth.Dims(n_vocab=500, n_text_ctx=32, n_text_state=128, n_text_head=2, n_text_layer=1, n_audio_ctx=64)
    TE = synth.make_encoder(edims, seed=8, qk_std=0.1)
    TD = synth.make_decoder(dims, seed=8)
    mel = synth.mel_input(edims, 8)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "m.bin")
        synth.write_ggml(path, dims, TD + TE, edims=edims)
        with gpu.Encoder.load_ggml(path) as ef:
            assert (ef.dims.n_mels, ef.dims.n_audio_ctx, ef.dims.n_audio_state, ef.dims.n_audio_head,
                    ef.dims.n_audio_layer) == (80, 64, 128, 2, 2)
            yf = ef.forward(mel)
        with gpu.Model.load_ggml(path) as m:  # the decoder loads from the same file
            assert m.dims.n_vocab == 500
    with gpu.Encoder.from_tensors(edims, TE) as et:
        yt = et.forward(mel)
    np.testing.assert_array_equal(yf, yt)


def test_encoder_to_decoder_on_device(gpu, orc):
    """mel -> encoder -> decoder without the host: w4h_encoder_forward_device writes xa into device
    memory and w4h_session_set_encoder_device takes it; the decoder's logits equal those of the same
    xa passed through host memory, bit for bit, and the whole chain agrees with oracle encoder +
    oracle decoder within the decoder's 1e-2 logit bar."""
    from whisper4j_amd.device import DeviceArray

    edims = synth.EncDims(80, 96, 256, 4, 2)
    dims = synth.Dims(n_vocab=700, n_text_ctx=32, n_text_state=256, n_text_head=4, n_text_layer=2, n_audio_ctx=96)
    TE = synth.make_encoder(edims, seed=9, qk_std=0.1)
    TD = synth.make_decoder(dims, seed=9)
    mel = synth.mel_input(edims, 9)
    with gpu.Encoder.from_tensors(edims, TE) as enc, gpu.Model.from_tensors(dims, TD) as model:
        xa_host = enc.forward(mel)
        with DeviceArray(mel) as dm, DeviceArray(np.zeros((96, 256), np.float32)) as dx:
            enc.forward_device(dm.address, dx.address)
            np.testing.assert_array_equal(dx.numpy(), xa_host)
            toks = [1, 2, 3, 4, 5]
            with model.session() as s1, model.session() as s2:
                s1.set_encoder_device(dx.address)
                s2.set_encoder(xa_host)
                for t in toks:
                    _, l1 = s1.step([t], want_logits=True)
                    _, l2 = s2.step([t], want_logits=True)
                    np.testing.assert_array_equal(l1, l2)
    oe = orc.Encoder(edims, TE)
    xa_ref = oe.forward(mel)
    oe.close()
    om = orc.Model(dims, TD)
    ref = om.forced(xa_ref, toks[:1], np.array(toks[1:], np.int32), want_logits=True)["logits"]
    err = float(np.abs(l1[0] - ref[-1]).max())
    say(f"encoder + decoder chain vs oracle: last-step max |d logit| {err:.2e}")
    assert err <= 1e-2


@pytest.mark.parametrize("name", ["tiny.en", "base.en"])
def test_encoder_full_size_against_fixture(gpu, name):
    """The encoder at its real size (80 mels x 3000 frames -> 1500 frames; tiny.en d 384 x 4 layers,
    base.en d 512 x 6 layers; seed-0 weights and mel) against the oracle's output written by
    tests/golden/make_encoder_fixture.py: 8 full rows within the element bar, and every frame's
    projection on 16 fixed N(0, 1) directions within 4e-3 * sqrt(d) (the element bar carried
    through a projection)."""
    import importlib.util

    here = os.path.dirname(os.path.abspath(__file__))
    spec = importlib.util.spec_from_file_location("mef", os.path.join(here, "golden", "make_encoder_fixture.py"))
    mef = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mef)
    fx = np.load(os.path.join(here, "golden", "encoder", f"{name}.npz"))
    ed = synth.ENC_SHAPES[name]
    T = synth.make_encoder(ed, seed=0)
    mel = synth.mel_input(ed, 0)
    with gpu.Encoder.from_tensors(ed, T) as enc:
        y = enc.forward(mel)
    _check(y[fx["rows_at"]], fx["rows"], f"{name} full size, sampled rows")
    p = y.astype(np.float64) @ mef.projection(ed.n_audio_state).astype(np.float64)
    dp = np.abs(p - fx["proj"])
    say(f"{name} projections: max |d| {dp.max():.2e} (bar {4e-3 * np.sqrt(ed.n_audio_state):.2e}), mean {dp.mean():.2e}")
    assert dp.max() <= 4e-3 * np.sqrt(ed.n_audio_state)
