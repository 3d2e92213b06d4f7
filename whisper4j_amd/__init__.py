"""whisper4j_amd: MI355X (gfx950) implementation of whisper4j's text-decoder token loop.

The decoder step runs as hand-written HIP kernels behind a C ABI (include/w4h.h, libw4h.so);
this package is the host-side mirror of the reference decoder interface plus the synthetic-model
generator used by the tests and the benchmark.
"""

from ._lib import EXPORTS, W4HError, device_count, lib  # noqa: F401
from .decoder import (  # noqa: F401
    DecodeResult,
    Encoder,
    Model,
    Session,
    StepResult,
    WhisperDecoder,
    compression_ratio,
    make_mask,
    op_attention,
    op_gelu,
    op_layernorm,
    op_linear,
    op_sample,
    op_select,
)
