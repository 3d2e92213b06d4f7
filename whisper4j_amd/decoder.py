"""Host-side mirror of whisper4j's decoder interface over the C ABI (libw4h.so).

``WhisperDecoder`` keeps the reference's method names and argument meaning
(``nn/WhisperDecoder.java:36, 59-204, 214-394``): ``forward``-style stepping through a session,
``decode``, ``decode_beam`` and ``decode_with_fallback`` returning a ``DecodeResult`` with the fields
of the reference record (``:672-673``).  Errors raise ``W4HError`` (the reference throws
IllegalArgumentException / IllegalStateException / IOException for the same conditions).
"""

from __future__ import annotations

import ctypes
import dataclasses

import numpy as np

from . import _lib
from ._lib import W4HError, check, lib

_i32p = ctypes.POINTER(ctypes.c_int32)
_f32p = ctypes.POINTER(ctypes.c_float)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u16p = ctypes.POINTER(ctypes.c_uint16)


def _ptr(a, t):
    return a.ctypes.data_as(t) if a is not None else None


@dataclasses.dataclass
class DecodeResult:
    tokens: list
    avg_logprob: float
    compression_ratio: float
    no_speech_prob: float
    temperature: float

    @classmethod
    def _from(cls, r: _lib.DecodeResult) -> "DecodeResult":
        return cls(list(r.tokens[: r.n_tokens]), r.avg_logprob, r.compression_ratio, r.no_speech_prob, r.temperature)


@dataclasses.dataclass
class StepResult:
    argmax: int
    max_logit: float
    logsumexp: float
    probe_logit: float
    raw_logsumexp: float
    topk_ids: list
    topk_logits: list

    @classmethod
    def _from(cls, o: _lib.StepOut, k: int) -> "StepResult":
        return cls(o.argmax, o.max_logit, o.logsumexp, o.probe_logit, o.raw_logsumexp, list(o.topk_ids[:k]),
                   list(o.topk_logits[:k]))


class Model:
    """Device-resident decoder weights (WhisperDecoder(WeightStore, ModelDimensions))."""

    def __init__(self, handle, dims: _lib.Dims):
        self._h = handle
        self.dims = dims

    @classmethod
    def from_tensors(cls, dims, tensors, device: int = 0) -> "Model":
        """dims: object with n_vocab, n_text_ctx, n_text_state, n_text_head, n_text_layer, n_audio_ctx;
        tensors: list of synth.GgmlTensor-like objects (name, ggml_type, ne, raw())."""
        d = _lib.Dims(dims.n_vocab, dims.n_text_ctx, dims.n_text_state, dims.n_text_head, dims.n_text_layer,
                      dims.n_audio_ctx)
        arr = (_lib.Tensor * len(tensors))()
        keep = []
        for i, t in enumerate(tensors):
            raw = np.ascontiguousarray(t.raw())
            nm = t.name.encode()
            keep += [raw, nm]
            arr[i].name = nm
            arr[i].type = t.ggml_type
            arr[i].n_dims = len(t.ne)
            for j, v in enumerate(t.ne):
                arr[i].ne[j] = int(v)
            arr[i].data = raw.ctypes.data
        h = ctypes.c_void_p()
        check(lib().w4h_model_create(ctypes.byref(d), arr, len(tensors), device, ctypes.byref(h)))
        return cls(h, d)

    @classmethod
    def load_ggml(cls, path: str, device: int = 0) -> "Model":
        h = ctypes.c_void_p()
        check(lib().w4h_model_load_ggml(path.encode(), device, ctypes.byref(h)))
        d = _lib.Dims()
        check(lib().w4h_model_dims(h, ctypes.byref(d)))
        return cls(h, d)

    def close(self) -> None:
        if self._h is not None:
            check(lib().w4h_model_destroy(self._h))
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def session(self, n_rows: int = 1, n_encoders: int = 1, max_ctx: int | None = None) -> "Session":
        return Session(self, n_rows, n_encoders, max_ctx or self.dims.n_text_ctx)


def _tensor_array(tensors):
    arr = (_lib.Tensor * len(tensors))()
    keep = []
    for i, t in enumerate(tensors):
        raw = np.ascontiguousarray(t.raw())
        nm = t.name.encode()
        keep += [raw, nm]
        arr[i].name = nm
        arr[i].type = t.ggml_type
        arr[i].n_dims = len(t.ne)
        for j, v in enumerate(t.ne):
            arr[i].ne[j] = int(v)
        arr[i].data = raw.ctypes.data
    return arr, keep


class Encoder:
    """Device-resident audio encoder (WhisperEncoder(WeightStore, ModelDimensions) and forward(mel),
    main/nn/WhisperEncoder.java:27-76)."""

    def __init__(self, handle, dims: _lib.EncoderDims):
        self._h = handle
        self.dims = dims

    @classmethod
    def from_tensors(cls, edims, tensors, device: int = 0) -> "Encoder":
        """edims: object with n_mels, n_audio_ctx, n_audio_state, n_audio_head, n_audio_layer."""
        d = _lib.EncoderDims(edims.n_mels, edims.n_audio_ctx, edims.n_audio_state, edims.n_audio_head,
                             edims.n_audio_layer)
        arr, keep = _tensor_array(tensors)
        h = ctypes.c_void_p()
        check(lib().w4h_encoder_create(ctypes.byref(d), arr, len(tensors), device, ctypes.byref(h)))
        del keep
        return cls(h, d)

    @classmethod
    def load_ggml(cls, path: str, device: int = 0) -> "Encoder":
        h = ctypes.c_void_p()
        check(lib().w4h_encoder_load_ggml(path.encode(), device, ctypes.byref(h)))
        d = _lib.EncoderDims()
        check(lib().w4h_encoder_get_dims(h, ctypes.byref(d)))
        return cls(h, d)

    def forward(self, mel) -> np.ndarray:
        """mel [n_mels][2 * n_audio_ctx] -> encoder output [n_audio_ctx][n_audio_state] (fp32)."""
        m = np.ascontiguousarray(mel, dtype=np.float32)
        if m.shape != (self.dims.n_mels, 2 * self.dims.n_audio_ctx):
            raise ValueError(f"mel shape {m.shape}, expected ({self.dims.n_mels}, {2 * self.dims.n_audio_ctx})")
        out = np.empty((self.dims.n_audio_ctx, self.dims.n_audio_state), np.float32)
        check(lib().w4h_encoder_forward(self._h, _ptr(m, _f32p), _ptr(out, _f32p)))
        return out

    def forward_device(self, mel_dev: int, out_dev: int, stream: int = 0) -> None:
        check(lib().w4h_encoder_forward_device(self._h, ctypes.c_void_p(mel_dev), ctypes.c_void_p(out_dev),
                                               ctypes.c_void_p(stream or None)))

    def close(self) -> None:
        if self._h is not None:
            check(lib().w4h_encoder_destroy(self._h))
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


class Session:
    """Per-decode-call state: self-KV cache, cross K/V, stream (the reference's kvCache map)."""

    def __init__(self, model: Model, n_rows: int, n_encoders: int, max_ctx: int):
        if model._h is None:
            raise W4HError(_lib.W4H_ERR_CLOSED, "model closed")
        self.model = model
        self.n_rows = n_rows
        self.vocab = model.dims.n_vocab
        desc = _lib.SessionDesc(n_rows, n_encoders, max_ctx)
        h = ctypes.c_void_p()
        check(lib().w4h_session_create(model._h, ctypes.byref(desc), ctypes.byref(h)))
        self._h = h

    def close(self) -> None:
        if self._h is not None:
            check(lib().w4h_session_destroy(self._h))
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def set_encoder(self, xa, enc: int = 0) -> None:
        xa = np.ascontiguousarray(xa, dtype=np.float32)
        check(lib().w4h_session_set_encoder(self._h, enc, _ptr(xa, _f32p)))

    def set_encoder_device(self, xa_ptr: int, enc: int = 0) -> None:
        """Encoder output already on the session's device: xa_ptr is the address of a contiguous
        fp32 [n_audio_ctx][n_text_state] buffer (e.g. a torch tensor's data_ptr()) whose producer
        has finished writing it."""
        check(lib().w4h_session_set_encoder_device(self._h, enc, ctypes.c_void_p(int(xa_ptr))))

    def reset(self, kv_len: int = 0) -> None:
        check(lib().w4h_session_reset(self._h, kv_len))

    def cancel(self, on: bool = True) -> None:
        """Request (on) or clear (off) cancellation; on may come from any thread (see w4h.h)."""
        check(lib().w4h_session_cancel(self._h, 1 if on else 0))

    @property
    def kv_len(self) -> int:
        n = ctypes.c_int32()
        check(lib().w4h_session_kv_len(self._h, ctypes.byref(n)))
        return n.value

    def set_suppress(self, ids) -> None:
        a = np.ascontiguousarray(list(ids), dtype=np.int32)
        check(lib().w4h_session_set_suppress(self._h, _ptr(a, _i32p), a.size))

    def set_probe(self, token: int) -> None:
        check(lib().w4h_session_set_probe(self._h, token))

    def set_logit_bias(self, bias) -> None:
        """Fixed bias [n_vocab] added to the raw logits of every row before selection (None: off)."""
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32).reshape(-1)
        if b is not None and b.size != self.vocab:
            raise ValueError(f"logit bias needs {self.vocab} values, got {b.size}")
        check(lib().w4h_session_set_logit_bias(self._h, _ptr(b, _f32p)))

    def step(self, tokens, extra_mask=None, topk: int = 0, want_logits: bool = False):
        t = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
        out = (_lib.StepOut * self.n_rows)()
        lg = np.empty((self.n_rows, self.vocab), np.float32) if want_logits else None
        m = np.ascontiguousarray(extra_mask, dtype=np.uint32) if extra_mask is not None else None
        check(lib().w4h_session_step(self._h, _ptr(t, _i32p), _ptr(m, _u32p), topk, out, _ptr(lg, _f32p)))
        res = [StepResult._from(out[i], topk) for i in range(self.n_rows)]
        return (res, lg) if want_logits else res

    def run(self, tokens, forced=None, n_steps: int = 1, topk: int = 0):
        t = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
        f = np.ascontiguousarray(forced, dtype=np.int32).reshape(-1) if forced is not None else None
        out = (_lib.StepOut * (n_steps * self.n_rows))()
        check(lib().w4h_session_run(self._h, _ptr(t, _i32p), _ptr(f, _i32p), n_steps, topk, out))
        return [[StepResult._from(out[i * self.n_rows + r], topk) for r in range(self.n_rows)] for i in range(n_steps)]

    def reorder(self, parent) -> None:
        p = np.ascontiguousarray(parent, dtype=np.int32)
        check(lib().w4h_session_reorder(self._h, _ptr(p, _i32p)))

    def time_run(self, tokens, forced, n_steps: int, n_repeats: int):
        t = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
        f = np.ascontiguousarray(forced, dtype=np.int32).reshape(-1) if forced is not None else None
        ms = np.zeros(n_repeats, np.float32)
        out = (_lib.StepOut * (n_steps * self.n_rows))()
        check(lib().w4h_session_time_run(self._h, _ptr(t, _i32p), _ptr(f, _i32p), n_steps, n_repeats, _ptr(ms, _f32p),
                                          out))
        return ms, [[StepResult._from(out[i * self.n_rows + r], 0) for r in range(self.n_rows)] for i in range(n_steps)]


def _phase_names(L):
    per = ["self_attn", "self_out", "cross_attn", "cross_out", "mlp1", "mlp2"]
    return [f"l{l}.{p}" for l in range(L) for p in per] + ["logits", "select"]


def trace_run(session: "Session", tokens, forced, n_steps: int):
    """Device timestamps -> (names, ticks[n_steps][n_phases][4][n_workgroups]); points per phase:
    0 entered, 1 inputs arrived, 2 computed, 3 left (0 where the workgroup had no work)."""
    t = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
    f = np.ascontiguousarray(forced, dtype=np.int32).reshape(-1) if forced is not None else None
    L = session.model.dims.n_text_layer
    nph = 6 * L + 2
    g = ctypes.c_int32()
    n = n_steps * nph * 4 * 1024
    buf = np.zeros(n, np.uint64)
    check(lib().w4h_session_trace_run(session._h, _ptr(t, _i32p), _ptr(f, _i32p), n_steps,
                                      buf.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)), n, ctypes.byref(g)))
    G = g.value
    return _phase_names(L), buf[: n_steps * nph * 4 * G].reshape(n_steps, nph, 4, G)


class WhisperDecoder:
    """Mirror of com.sparrowlogic.whisper4j.nn.WhisperDecoder running on the device."""

    def __init__(self, model: Model, beam_size: int = 1, max_ctx: int | None = None):
        self.model = model
        self.session = model.session(n_rows=max(1, beam_size), n_encoders=1, max_ctx=max_ctx)
        self._xa_id = None

    def close(self):
        self.session.close()

    def set_logit_bias(self, bias) -> None:
        self.session.set_logit_bias(bias)

    def _opts(self, prompt, eot, max_tokens, suppress, no_speech, temperature, timestamp_begin, beam_size, seed):
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        s = np.ascontiguousarray(list(suppress or []), dtype=np.int32)
        o = _lib.DecodeOpts(_ptr(p, _i32p), p.size, eot, max_tokens, _ptr(s, _i32p), s.size, no_speech,
                            float(temperature), timestamp_begin, beam_size, seed)
        return o, (p, s)

    def _encoder(self, encoder_output):
        xa = np.ascontiguousarray(encoder_output, dtype=np.float32)
        key = (xa.ctypes.data, xa.shape, hash(xa[:: max(1, xa.shape[0] // 7)].tobytes()))
        if key != self._xa_id:
            self.session.set_encoder(xa.reshape(-1, self.model.dims.n_text_state))
            self._xa_id = key

    def decode(self, encoder_output, prompt, eot_token, max_tokens, suppress_tokens=(), no_speech_token=-1,
               temperature=0.0, timestamp_begin=-1, seed=0) -> DecodeResult:
        self._encoder(encoder_output)
        o, keep = self._opts(prompt, eot_token, max_tokens, suppress_tokens, no_speech_token, temperature,
                             timestamp_begin, 1, seed)
        r = _lib.DecodeResult()
        check(lib().w4h_decode(self.session._h, ctypes.byref(o), ctypes.byref(r)))
        return DecodeResult._from(r)

    def decode_beam(self, encoder_output, prompt, eot_token, max_tokens, suppress_tokens=(), no_speech_token=-1,
                    timestamp_begin=-1, beam_size=5) -> DecodeResult:
        self._encoder(encoder_output)
        o, keep = self._opts(prompt, eot_token, max_tokens, suppress_tokens, no_speech_token, 0.0, timestamp_begin,
                             beam_size, 0)
        r = _lib.DecodeResult()
        check(lib().w4h_decode_beam(self.session._h, ctypes.byref(o), ctypes.byref(r)))
        return DecodeResult._from(r)

    def decode_with_fallback(self, encoder_output, prompt, eot_token, max_tokens, suppress_tokens=(),
                             no_speech_token=-1, timestamp_begin=-1, beam_size=1, seed=0) -> DecodeResult:
        self._encoder(encoder_output)
        o, keep = self._opts(prompt, eot_token, max_tokens, suppress_tokens, no_speech_token, 0.0, timestamp_begin,
                             beam_size, seed)
        r = _lib.DecodeResult()
        check(lib().w4h_decode_with_fallback(self.session._h, ctypes.byref(o), ctypes.byref(r)))
        return DecodeResult._from(r)


def compression_ratio(tokens) -> float:
    t = np.ascontiguousarray(tokens, dtype=np.int32)
    r = ctypes.c_float()
    check(lib().w4h_compression_ratio(_ptr(t, _i32p), t.size, ctypes.byref(r)))
    return r.value


# ---- kernel-level entry points ------------------------------------------------------------

def op_linear(w_raw, w_type: int, n: int, k: int, x, bias=None):
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    w_raw = np.ascontiguousarray(w_raw)
    b = np.ascontiguousarray(bias, dtype=np.float32) if bias is not None else None
    y = np.empty((x.shape[0], n), np.float32)
    check(lib().w4h_op_linear(w_raw.ctypes.data, w_type, n, k, _ptr(b, _f32p), _ptr(x, _f32p), x.shape[0],
                              _ptr(y, _f32p)))
    return y


def op_layernorm(x, gamma, beta):
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    g = np.ascontiguousarray(gamma, dtype=np.float32)
    b = np.ascontiguousarray(beta, dtype=np.float32)
    y = np.empty_like(x)
    check(lib().w4h_op_layernorm(_ptr(x, _f32p), x.shape[0], x.shape[1], _ptr(g, _f32p), _ptr(b, _f32p), _ptr(y, _f32p)))
    return y


def op_gelu(x):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    y = np.empty_like(x)
    check(lib().w4h_op_gelu(_ptr(x, _f32p), x.size, _ptr(y, _f32p)))
    return y


def op_attention(q, k_f16, v_f16, scale=0.125):
    """q [H][64] fp32; k, v [H][L][64] float16 arrays."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k_f16, dtype=np.float16).view(np.uint16)
    v = np.ascontiguousarray(v_f16, dtype=np.float16).view(np.uint16)
    out = np.empty_like(q)
    check(lib().w4h_op_attention(_ptr(q, _f32p), _ptr(k, _u16p), _ptr(v, _u16p), q.shape[0], k.shape[1],
                                 ctypes.c_float(scale), _ptr(out, _f32p)))
    return out


def op_select(logits, k=0, mask=None):
    lg = np.ascontiguousarray(np.atleast_2d(logits), dtype=np.float32)
    m = np.ascontiguousarray(mask, dtype=np.uint32) if mask is not None else None
    out = (_lib.StepOut * lg.shape[0])()
    check(lib().w4h_op_select(_ptr(lg, _f32p), lg.shape[0], lg.shape[1], _ptr(m, _u32p), k, out))
    return [StepResult._from(out[i], k) for i in range(lg.shape[0])]


def op_sample(logits, temperature, rng_state, history=(), eot=0, timestamp_begin=-1, suppress_mask=None):
    """The device sampling step of a T > 0 decode on one row: (token, log-probability)."""
    lg = np.ascontiguousarray(logits, dtype=np.float32).ravel()
    m = np.ascontiguousarray(suppress_mask, dtype=np.uint32).ravel() if suppress_mask is not None else None
    h = np.ascontiguousarray(list(history) or [0], dtype=np.int32)
    tok, lp = ctypes.c_int32(0), ctypes.c_double(0.0)
    check(lib().w4h_op_sample(_ptr(lg, _f32p), lg.size, _ptr(m, _u32p), _ptr(h, _i32p), len(history), eot,
                              timestamp_begin, ctypes.c_float(temperature), ctypes.c_uint64(rng_state),
                              ctypes.byref(tok), ctypes.byref(lp)))
    return int(tok.value), float(lp.value)


def make_mask(rows: int, vocab: int, ids_per_row) -> np.ndarray:
    """Bitmask [rows][ceil(vocab/32)] with the listed token ids set."""
    mw = (vocab + 31) // 32
    m = np.zeros((rows, mw), np.uint32)
    for r, ids in enumerate(ids_per_row):
        for t in ids:
            if 0 <= t < vocab:
                m[r, t >> 5] |= np.uint32(1 << (t & 31))
    return m
