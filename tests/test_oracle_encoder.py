"""Pins the oracle's audio encoder (WhisperEncoder, main/nn/WhisperEncoder.java:42-76; Conv1d,
main/nn/Conv1d.java:38-80) against closed forms and an independent float64 formulation:
- Conv1d against the definition y[o][t] = b[o] + sum_{i,k} w[o][i][k] x[i][s t - p + k] in float64,
  within the float32 summation bound, for stride 1 and 2, with the zero padding at both ends;
- the whole encoder (f16 and q8_0 matrices) against tests/np_encoder.py within 2e-3 (LayerNorm
  outputs of unit scale; float32 rounding, plus the f16 index of GELU inputs that sit on a rounding
  edge), with peaked attention (query/key weights N(0, 0.1)) so that a wrong softmax axis, scale,
  head split or residual would show."""

import numpy as np
import pytest

from tests.np_encoder import encoder_forward
from whisper4j_amd import synth


@pytest.mark.parametrize("stride,in_ch,n", [(1, 80, 37), (2, 64, 40), (2, 8, 7)])
def test_conv1d_definition(orc, stride, in_ch, n):
    rng = np.random.default_rng(stride * 100 + n)
    out_ch = 24
    w = rng.standard_normal((out_ch, in_ch, 3)).astype(np.float32)
    b = rng.standard_normal(out_ch).astype(np.float32)
    x = rng.standard_normal((in_ch, n)).astype(np.float32)
    y = orc.conv1d(w, b, stride, 1, x)
    out_len = (n + 2 - 3) // stride + 1
    assert y.shape == (out_ch, out_len)
    ref = np.zeros((out_ch, out_len))
    bound = np.zeros((out_ch, out_len))
    w64, x64 = w.astype(np.float64), x.astype(np.float64)
    for t in range(out_len):
        for k in range(3):
            j = stride * t - 1 + k
            if 0 <= j < n:
                ref[:, t] += w64[:, :, k] @ x64[:, j]
                bound[:, t] += np.abs(w64[:, :, k]) @ np.abs(x64[:, j])
    ref += b[:, None]
    gamma = 3 * in_ch * 2.0 ** -24 / (1 - 3 * in_ch * 2.0 ** -24)
    assert np.all(np.abs(y - ref) <= gamma * bound + 2.0 ** -23 * (np.abs(ref) + np.abs(b)[:, None]))


@pytest.mark.parametrize("wtype,edims", [
    ("f16", synth.EncDims(80, 48, 128, 2, 2)),
    ("q8_0", synth.EncDims(16, 40, 128, 2, 1)),
    ("f16", synth.EncDims(128, 33, 192, 3, 1)),
])
def test_encoder_matches_float64(orc, wtype, edims):
    T = synth.make_encoder(edims, seed=3, wtype=wtype, ln_random=True, qk_std=0.1)
    mel = synth.mel_input(edims, 3)
    e = orc.Encoder(edims, T)
    y = e.forward(mel)
    e.close()
    ref = encoder_forward(edims, T, mel)
    err = np.abs(y - ref)
    assert y.shape == (edims.n_audio_ctx, edims.n_audio_state)
    assert err.max() < 2e-3, err.max()
    assert err.mean() < 2e-4, err.mean()
