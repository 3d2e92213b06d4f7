"""Seeded synthetic Whisper text-decoder weights and inputs, in GGML tensor form.

The decoder shapes are the five Whisper-family shapes the benchmark and parity tests use.
Weights follow the GGML/whisper.cpp tensor names and layouts that the reference loader reads
(``model/GgmlLoader.java:148-216``): 2-D matrices are ``[out][in]`` row-major (GGML ``ne = [in, out]``),
stored f16 or q8_0; biases, LayerNorm parameters and the positional embedding are f32.

Generation: each tensor draws from ``numpy.random.default_rng([seed, crc32(name)])`` (PCG64), so a
tensor's values depend only on the global seed and its name.  Matrices and biases are N(0, 0.02),
LayerNorm gamma = 1 and beta = 0, the encoder output is N(0, 1) fp32 ``[n_audio_ctx, d]``.
q8_0 follows GGML's published quantizer: per 32-element block along K, ``d = amax / 127`` stored as
f16 and ``q = roundf(x / d)`` as int8.
"""

from __future__ import annotations

import dataclasses
import struct
import zlib

import numpy as np

GGML_F32 = 0
GGML_F16 = 1
GGML_Q8_0 = 8
GGML_MAGIC = 0x67676D6C

# Prompt used by every benchmark configuration: <|endoftext|> <|startoftranscript|> ... as in the
# reference's stage validation harness.
BENCH_PREFIX = (50257, 50258, 50359, 50363)
# <|endoftext|> of the multilingual vocabulary (51865 ids), the end token of the beam workload
EOT_MULTILINGUAL = 50257
BEAM_BIAS_SIGMA = 1.0


@dataclasses.dataclass(frozen=True)
class Dims:
    n_vocab: int
    n_text_ctx: int
    n_text_state: int
    n_text_head: int
    n_text_layer: int
    n_audio_ctx: int = 1500

    @property
    def n_mlp(self) -> int:
        return 4 * self.n_text_state


SHAPES = {
    "tiny.en": Dims(51864, 448, 384, 6, 4),
    "base.en": Dims(51864, 448, 512, 8, 6),
    "small": Dims(51865, 448, 768, 12, 12),
    "large-v3-turbo": Dims(51866, 448, 1280, 20, 4),
    "medium": Dims(51865, 448, 1024, 16, 24),
}


@dataclasses.dataclass(frozen=True)
class EncDims:
    """Audio encoder hyperparameters (WhisperEncoder, main/nn/WhisperEncoder.java:27-38)."""
    n_mels: int
    n_audio_ctx: int
    n_audio_state: int
    n_audio_head: int
    n_audio_layer: int


ENC_SHAPES = {
    "tiny.en": EncDims(80, 1500, 384, 6, 4),
    "base.en": EncDims(80, 1500, 512, 8, 6),
    "small": EncDims(80, 1500, 768, 12, 12),
    "large-v3-turbo": EncDims(128, 1500, 1280, 20, 32),
    "medium": EncDims(80, 1500, 1024, 16, 24),
}


@dataclasses.dataclass
class GgmlTensor:
    name: str
    ggml_type: int
    ne: tuple  # GGML order: ne[0] is the contiguous dimension
    data: np.ndarray  # raw bytes as uint8 (q8_0) or typed array (f32/f16), C-contiguous

    @property
    def numel(self) -> int:
        n = 1
        for v in self.ne:
            n *= int(v)
        return n

    def raw(self) -> np.ndarray:
        return np.ascontiguousarray(self.data).view(np.uint8).reshape(-1)


def _rng(seed: int, name: str) -> np.random.Generator:
    return np.random.default_rng([int(seed) & 0xFFFFFFFF, zlib.crc32(name.encode())])


def quantize_q8_0(w: np.ndarray) -> np.ndarray:
    """GGML quantize_row_q8_0 on rows of a [N][K] matrix (K % 32 == 0) -> raw 34-byte blocks."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    if w.shape[-1] % 32:
        raise ValueError("q8_0 needs K % 32 == 0")
    blocks = w.reshape(-1, 32)
    amax = np.max(np.abs(blocks), axis=1)
    d = amax / 127.0
    idv = np.where(d != 0, 1.0 / np.where(d != 0, d, 1.0), 0.0).astype(np.float32)
    xs = blocks * idv[:, None]
    q = (np.sign(xs) * np.floor(np.abs(xs) + 0.5)).astype(np.int8)  # roundf: half away from zero
    out = np.empty((blocks.shape[0], 34), dtype=np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def dequantize_q8_0(raw: np.ndarray, numel: int) -> np.ndarray:
    """Inverse of the storage format (GgmlLoader.dequantizeQ8_0, model/GgmlLoader.java:292-300)."""
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 34)[: numel // 32]
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1)
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (q * d[:, None]).reshape(-1)


def tensor_to_f32(t: GgmlTensor) -> np.ndarray:
    """Dequantize any supported tensor to fp32, shaped row-major (reversed ne)."""
    shape = tuple(int(v) for v in reversed(t.ne))
    if t.ggml_type == GGML_F32:
        return np.asarray(t.data, dtype=np.float32).reshape(shape)
    if t.ggml_type == GGML_F16:
        return np.asarray(t.data, dtype=np.float16).astype(np.float32).reshape(shape)
    if t.ggml_type == GGML_Q8_0:
        return dequantize_q8_0(t.data, t.numel).reshape(shape)
    raise ValueError(f"unsupported ggml type {t.ggml_type}")


def _matrix(seed, name, n_out, n_in, wtype, std=0.02):
    w = (_rng(seed, name).standard_normal((n_out, n_in), dtype=np.float32) * np.float32(std))
    if wtype == "f16":
        return GgmlTensor(name, GGML_F16, (n_in, n_out), w.astype(np.float16))
    if wtype == "q8_0":
        return GgmlTensor(name, GGML_Q8_0, (n_in, n_out), quantize_q8_0(w))
    if wtype == "f32":
        return GgmlTensor(name, GGML_F32, (n_in, n_out), w)
    raise ValueError(wtype)


def _vector(seed, name, n, kind):
    if kind == "ones":
        v = np.ones(n, dtype=np.float32)
    elif kind == "zeros":
        v = np.zeros(n, dtype=np.float32)
    else:
        v = _rng(seed, name).standard_normal(n, dtype=np.float32) * np.float32(0.02)
    return GgmlTensor(name, GGML_F32, (n,), v)


def make_decoder(dims: Dims, seed: int = 0, wtype: str = "f16", ln_random: bool = False) -> list:
    """Tensor table of a random-init Whisper text decoder (names as whisper.cpp / the reference).

    ``ln_random`` draws LayerNorm gamma/beta from N(1, 0.1)/N(0, 0.1) instead of 1/0 so tests can
    tell gamma from beta.
    """
    d, V, C, L = dims.n_text_state, dims.n_vocab, dims.n_text_ctx, dims.n_text_layer
    out = [
        _matrix(seed, "decoder.token_embedding.weight", V, d, wtype),
        GgmlTensor(
            "decoder.positional_embedding",
            GGML_F32,
            (d, C),
            _rng(seed, "decoder.positional_embedding").standard_normal((C, d), dtype=np.float32) * np.float32(0.02),
        ),
    ]

    def ln(name):
        if ln_random:
            g = 1.0 + 0.1 * _rng(seed, name + ".weight").standard_normal(d, dtype=np.float32)
            b = 0.1 * _rng(seed, name + ".bias").standard_normal(d, dtype=np.float32)
            return [GgmlTensor(name + ".weight", GGML_F32, (d,), g.astype(np.float32)),
                    GgmlTensor(name + ".bias", GGML_F32, (d,), b.astype(np.float32))]
        return [_vector(seed, name + ".weight", d, "ones"), _vector(seed, name + ".bias", d, "zeros")]

    out += ln("decoder.ln")
    for i in range(L):
        p = f"decoder.blocks.{i}."
        for a in ("attn", "cross_attn"):
            for proj in ("query", "key", "value", "out"):
                out.append(_matrix(seed, f"{p}{a}.{proj}.weight", d, d, wtype))
                if proj != "key":
                    out.append(_vector(seed, f"{p}{a}.{proj}.bias", d, "normal"))
        out += ln(p + "attn_ln") + ln(p + "cross_attn_ln") + ln(p + "mlp_ln")
        out.append(_matrix(seed, p + "mlp.0.weight", 4 * d, d, wtype))
        out.append(_vector(seed, p + "mlp.0.bias", 4 * d, "normal"))
        out.append(_matrix(seed, p + "mlp.2.weight", d, 4 * d, wtype))
        out.append(_vector(seed, p + "mlp.2.bias", d, "normal"))
    return out


def make_encoder(edims: EncDims, seed: int = 0, wtype: str = "f16", ln_random: bool = False,
                 qk_std: float = 0.02) -> list:
    """Tensor table of a random-init Whisper audio encoder (names and GGML shapes as whisper.cpp):
    conv weights f16 [out][in][3] (ne = [3, in, out]), conv biases f32 ne = [1, out], the positional
    embedding f32 [n_audio_ctx][d], blocks as the decoder's without cross-attention, ln_post.  The
    query and key matrices draw N(0, qk_std) (a larger value gives peaked attention)."""
    d, T, nm, L = edims.n_audio_state, edims.n_audio_ctx, edims.n_mels, edims.n_audio_layer

    def conv(name, n_out, n_in):
        w = _rng(seed, name).standard_normal((n_out, n_in, 3), dtype=np.float32) * np.float32(0.02)
        return GgmlTensor(name, GGML_F16, (3, n_in, n_out), w.astype(np.float16))

    def bias2(name, n):
        v = _rng(seed, name).standard_normal(n, dtype=np.float32) * np.float32(0.02)
        return GgmlTensor(name, GGML_F32, (1, n), v)

    def ln(name):
        if ln_random:
            g = 1.0 + 0.1 * _rng(seed, name + ".weight").standard_normal(d, dtype=np.float32)
            b = 0.1 * _rng(seed, name + ".bias").standard_normal(d, dtype=np.float32)
            return [GgmlTensor(name + ".weight", GGML_F32, (d,), g.astype(np.float32)),
                    GgmlTensor(name + ".bias", GGML_F32, (d,), b.astype(np.float32))]
        return [_vector(seed, name + ".weight", d, "ones"), _vector(seed, name + ".bias", d, "zeros")]

    out = [conv("encoder.conv1.weight", d, nm), bias2("encoder.conv1.bias", d),
           conv("encoder.conv2.weight", d, d), bias2("encoder.conv2.bias", d),
           GgmlTensor("encoder.positional_embedding", GGML_F32, (d, T),
                      _rng(seed, "encoder.positional_embedding").standard_normal((T, d), dtype=np.float32) * np.float32(0.02))]
    for i in range(L):
        p = f"encoder.blocks.{i}."
        for proj in ("query", "key", "value", "out"):
            std = qk_std if proj in ("query", "key") else 0.02
            out.append(_matrix(seed, f"{p}attn.{proj}.weight", d, d, wtype, std=std))
            if proj != "key":
                out.append(_vector(seed, f"{p}attn.{proj}.bias", d, "normal"))
        out += ln(p + "attn_ln") + ln(p + "mlp_ln")
        out.append(_matrix(seed, p + "mlp.0.weight", 4 * d, d, wtype))
        out.append(_vector(seed, p + "mlp.0.bias", 4 * d, "normal"))
        out.append(_matrix(seed, p + "mlp.2.weight", d, 4 * d, wtype))
        out.append(_vector(seed, p + "mlp.2.bias", d, "normal"))
    out += ln("encoder.ln_post")
    return out


def mel_input(edims: EncDims, seed: int = 0) -> np.ndarray:
    """A synthetic log-mel input [n_mels][2 * n_audio_ctx], N(0, 0.6) fp32."""
    return _rng(seed, "mel").standard_normal((edims.n_mels, 2 * edims.n_audio_ctx), dtype=np.float32) * np.float32(0.6)


def encoder_output(dims: Dims, seed: int = 0, stream: int = 0) -> np.ndarray:
    return _rng(seed, f"encoder_output.{stream}").standard_normal((dims.n_audio_ctx, dims.n_text_state),
                                                                  dtype=np.float32)


def logit_bias(dims: Dims, seed: int = 0, sigma: float = 1.0, eot: int | None = None) -> np.ndarray:
    """The beam workload's fixed logit bias: N(0, sigma) per vocabulary id, the end token at -inf so
    every hypothesis runs the full step count."""
    b = _rng(seed, "logit_bias").standard_normal(dims.n_vocab, dtype=np.float32) * np.float32(sigma)
    if eot is not None:
        b[eot] = -np.inf
    return b


def forced_tokens(n: int, seed: int = 0, high: int = 50256) -> np.ndarray:
    """Teacher-forced token IDs, uniform in [0, high]."""
    return _rng(seed, "forced_tokens").integers(0, high + 1, size=n, dtype=np.int32)


def write_ggml(path: str, dims: Dims, tensors: list, ftype: int = 1, edims: EncDims | None = None) -> None:
    """Write a whisper.cpp GGML file (layout read by model/GgmlLoader.java:95-216).

    Without ``edims`` the file carries placeholder encoder hparams; there are no mel filters and no
    vocab.
    """
    with open(path, "wb") as f:
        f.write(struct.pack("<i", GGML_MAGIC))
        if edims is None:
            enc = [dims.n_audio_ctx, dims.n_text_state, dims.n_text_head, 0, 80]
        else:
            enc = [edims.n_audio_ctx, edims.n_audio_state, edims.n_audio_head, edims.n_audio_layer, edims.n_mels]
        hp = [dims.n_vocab, enc[0], enc[1], enc[2], enc[3],
              dims.n_text_ctx, dims.n_text_state, dims.n_text_head, dims.n_text_layer, enc[4], ftype]
        f.write(struct.pack("<11i", *hp))
        f.write(struct.pack("<ii", 0, 0))  # mel filters: n_mel, n_fft
        f.write(struct.pack("<i", 0))  # vocab count
        for t in tensors:
            name = t.name.encode()
            f.write(struct.pack("<iii", len(t.ne), len(name), t.ggml_type))
            f.write(struct.pack(f"<{len(t.ne)}i", *[int(v) for v in t.ne]))
            f.write(name)
            f.write(t.raw().tobytes())
