"""Writes the oracle's audio-encoder output at full size as a fixture for the GPU parity test.

The workload is the benchmark's encoder: the tiny.en and base.en encoder shapes (80 mels, 1500
frames; d 384 / 512, 4 / 6 layers), seed-0 weights from whisper4j_amd.synth.make_encoder (f16) and
the seed-0 mel input [80][3000].  The oracle (oracle/libwhisper_ref.so, the CPU restatement of
WhisperEncoder.forward) runs here, in the build container; only its results are kept, compactly:

  rows   the full output rows of 8 frames (first, middle, last and neighbours)
  proj   every frame's output projected on 16 fixed N(0, 1) directions ([1500][16], seed 1234), which
         covers all 1500 x d values at once

Usage (about a minute):  python tests/golden/make_encoder_fixture.py
"""

from __future__ import annotations

import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT = os.path.join(HERE, "encoder")
sys.path.insert(0, ROOT)

from whisper4j_amd import synth  # noqa: E402

SHAPES = ("tiny.en", "base.en")
ROWS = (0, 1, 2, 749, 750, 1497, 1498, 1499)
NPROJ, PROJ_SEED = 16, 1234


def projection(d: int) -> np.ndarray:
    return np.random.default_rng(PROJ_SEED).standard_normal((d, NPROJ)).astype(np.float32)


def main() -> None:
    from oracle import oracle as orc

    os.makedirs(OUT, exist_ok=True)
    for name in SHAPES:
        ed = synth.ENC_SHAPES[name]
        t0 = time.time()
        T = synth.make_encoder(ed, seed=0)
        mel = synth.mel_input(ed, 0)
        e = orc.Encoder(ed, T)
        y = e.forward(mel)
        e.close()
        np.savez_compressed(os.path.join(OUT, f"{name}.npz"), rows_at=np.array(ROWS, np.int32), rows=y[list(ROWS)],
                            proj=(y.astype(np.float64) @ projection(ed.n_audio_state).astype(np.float64)).astype(np.float32))
        print(f"{name}: {time.time() - t0:.1f} s", flush=True)


if __name__ == "__main__":
    main()
