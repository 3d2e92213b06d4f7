"""ctypes wrapper of the oracle (libwhisper_ref.so, a CPU restatement of whisper4j's decode path).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline
leg, always as the parity reference (or the timed CPU baseline), never by the product package.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libwhisper_ref.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)


class OrcTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_int32), ("n_dims", ctypes.c_int32),
                ("ne", ctypes.c_int64 * 4), ("data", ctypes.c_void_p)]


class OrcDims(ctypes.Structure):
    _fields_ = [("n_vocab", ctypes.c_int32), ("n_text_ctx", ctypes.c_int32), ("n_text_state", ctypes.c_int32),
                ("n_text_head", ctypes.c_int32), ("n_text_layer", ctypes.c_int32), ("n_audio_ctx", ctypes.c_int32)]


class OrcEncDims(ctypes.Structure):
    _fields_ = [("n_mels", ctypes.c_int32), ("n_audio_ctx", ctypes.c_int32), ("n_audio_state", ctypes.c_int32),
                ("n_audio_head", ctypes.c_int32), ("n_audio_layer", ctypes.c_int32)]


class OrcResult(ctypes.Structure):
    _fields_ = [("n_tokens", ctypes.c_int32), ("tokens", ctypes.c_int32 * 1024), ("avg_logprob", ctypes.c_float),
                ("compression_ratio", ctypes.c_float), ("no_speech_prob", ctypes.c_float),
                ("temperature", ctypes.c_float)]

    def as_dict(self):
        return {"tokens": list(self.tokens[: self.n_tokens]), "avg_logprob": self.avg_logprob,
                "compression_ratio": self.compression_ratio, "no_speech_prob": self.no_speech_prob,
                "temperature": self.temperature}


_PREFILL = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, _f32p, _f32p)
_STEP = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int32, _f32p)
_REARRANGE = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, _i32p, ctypes.c_int, ctypes.c_int)


class OrcOps(ctypes.Structure):
    _fields_ = [("ctx", ctypes.c_void_p), ("prefill", _PREFILL), ("step", _STEP), ("rearrange", _REARRANGE)]


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_dot.restype = ctypes.c_float
        L.orc_dot.argtypes = [_f32p, _f32p, ctypes.c_int]
        L.orc_compression_ratio.restype = ctypes.c_float
        L.orc_argmax.restype = ctypes.c_int
        L.orc_dequant_q8_0.argtypes = [ctypes.c_void_p, ctypes.c_int64, _f32p]
        L.orc_model_create.restype = ctypes.c_void_p
        L.orc_model_create.argtypes = [ctypes.POINTER(OrcDims), ctypes.POINTER(OrcTensor), ctypes.c_int,
                                       ctypes.c_char_p, ctypes.c_int]
        L.orc_model_destroy.argtypes = [ctypes.c_void_p]
        L.orc_cache_create.restype = ctypes.c_void_p
        L.orc_cache_create.argtypes = [ctypes.c_void_p]
        L.orc_cache_destroy.argtypes = [ctypes.c_void_p]
        L.orc_cache_len.argtypes = [ctypes.c_void_p]
        L.orc_forward.argtypes = [ctypes.c_void_p, _i32p, ctypes.c_int, _f32p, ctypes.c_void_p, _f32p]
        L.orc_decode.argtypes = [ctypes.c_void_p, _f32p, _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _i32p,
                                 ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_uint64,
                                 ctypes.POINTER(OrcResult)]
        L.orc_decode_beam.argtypes = [ctypes.c_void_p, _f32p, _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _i32p,
                                      ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      ctypes.POINTER(OrcResult)]
        L.orc_decode_with_fallback.argtypes = [ctypes.c_void_p, _f32p, _i32p, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_int, _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_int, ctypes.c_uint64, ctypes.POINTER(OrcResult)]
        L.orc_forced.argtypes = [ctypes.c_void_p, _f32p, _i32p, ctypes.c_int, _i32p, ctypes.c_int, _i32p, _f32p,
                                 _f32p, _f32p, _f32p]
        L.orc_model_set_logit_bias.argtypes = [ctypes.c_void_p, _f32p]
        L.orc_suppress_blank.argtypes = [_f32p, ctypes.c_int, ctypes.c_int]
        L.orc_apply_suppress.argtypes = [_f32p, _i32p, ctypes.c_int, ctypes.c_int]
        L.orc_ngram_block.argtypes = [_f32p, _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.orc_timestamp_rules.argtypes = [_f32p, _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int]
        L.orc_needs_fallback.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_float]
        L.orc_sample_u.argtypes = [_f32p, ctypes.c_int, ctypes.c_float, ctypes.c_double]
        L.orc_encoder_create.restype = ctypes.c_void_p
        L.orc_encoder_create.argtypes = [ctypes.POINTER(OrcEncDims), ctypes.POINTER(OrcTensor), ctypes.c_int,
                                         ctypes.c_char_p, ctypes.c_int]
        L.orc_encoder_destroy.argtypes = [ctypes.c_void_p]
        L.orc_encoder_forward.restype = ctypes.c_int
        L.orc_encoder_forward.argtypes = [ctypes.c_void_p, _f32p, _f32p]
        L.orc_conv1d.argtypes = [_f32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 _f32p, ctypes.c_int, _f32p]
        L.orc_log_softmax_at.restype = ctypes.c_double
        L.orc_log_softmax_at.argtypes = [_f32p, ctypes.c_int, ctypes.c_int]
        L.orc_splitmix64_next.restype = ctypes.c_uint64
        L.orc_splitmix64_next.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        L.orc_rng_uniform.restype = ctypes.c_double
        L.orc_rng_uniform.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        L.orc_fallback_pick.argtypes = [ctypes.POINTER(OrcResult), ctypes.POINTER(ctypes.c_int)]
        L.orc_greedy_drive.argtypes = [ctypes.POINTER(OrcOps), ctypes.c_int, ctypes.c_int, ctypes.c_int, _i32p,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_uint64,
                                       ctypes.POINTER(OrcResult)]
        L.orc_beam_drive.argtypes = [ctypes.POINTER(OrcOps), ctypes.c_int, ctypes.c_int, ctypes.c_int, _i32p,
                                     ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(OrcResult),
                                     ctypes.POINTER(ctypes.c_double)]
        L.orc_decode_beam_gaps.argtypes = [ctypes.c_void_p, _f32p, _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                           _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                           ctypes.POINTER(OrcResult), ctypes.POINTER(ctypes.c_double)]
        _lib = L
    return _lib


def _p(a, t=_f32p):
    return a.ctypes.data_as(t) if a is not None else None


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


# ---- elementary ops --------------------------------------------------------------------------

def gelu_table() -> np.ndarray:
    t = np.empty(65536, dtype=np.float32)
    lib().orc_gelu_table(_p(t))
    return t


def gelu(x) -> np.ndarray:
    y = f32(x).copy()
    lib().orc_gelu(_p(y), ctypes.c_int(y.size))
    return y


def dot(a, b) -> float:
    a, b = f32(a), f32(b)
    return float(lib().orc_dot(_p(a), _p(b), a.size))


def layernorm(x, g, b, eps=1e-5) -> np.ndarray:
    x = f32(x)
    rows, n = (1, x.size) if x.ndim == 1 else x.shape
    out = np.empty_like(x)
    lib().orc_layernorm(_p(x), ctypes.c_int(rows), ctypes.c_int(n), _p(f32(g)), _p(f32(b)), ctypes.c_float(eps),
                        _p(out))
    return out


def linear(x, w, bias=None) -> np.ndarray:
    """y = x @ w.T + bias with the reference's Linear arithmetic; w is [out][in]."""
    x = f32(np.atleast_2d(x))
    w = f32(w)
    wt = f32(w.T)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n), dtype=np.float32)
    bb = f32(bias) if bias is not None else None
    lib().orc_linear(_p(x), ctypes.c_int(m), ctypes.c_int(k), _p(wt), ctypes.c_int(n), _p(bb), _p(y))
    return y


def attention_head(q, k, v, scale=0.125) -> np.ndarray:
    q, k, v = f32(q), f32(k), f32(v)
    out = np.empty(q.size, dtype=np.float32)
    lib().orc_attention_head(_p(q), _p(k), _p(v), ctypes.c_int(k.shape[0]), ctypes.c_int(q.size),
                             ctypes.c_float(scale), _p(out))
    return out


def softmax_rows(x) -> np.ndarray:
    y = f32(np.atleast_2d(x)).copy()
    lib().orc_softmax_rows(_p(y), ctypes.c_int(y.shape[0]), ctypes.c_int(y.shape[1]))
    return y


def argmax(a) -> int:
    a = f32(a)
    return int(lib().orc_argmax(_p(a), ctypes.c_int(a.size)))


def log_softmax(a) -> np.ndarray:
    a = f32(a)
    out = np.empty_like(a)
    lib().orc_log_softmax(_p(a), ctypes.c_int(a.size), _p(out))
    return out


def topk(a, k) -> list:
    a = f32(a)
    idx = np.empty(k, dtype=np.int32)
    lib().orc_topk(_p(a), ctypes.c_int(a.size), ctypes.c_int(k), _p(idx, _i32p))
    return idx.tolist()


def compression_ratio(tokens) -> float:
    t = i32(tokens)
    return float(lib().orc_compression_ratio(_p(t, _i32p), ctypes.c_int(t.size)))


def dequant_q8_0(raw, n: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(n, np.float32)
    lib().orc_dequant_q8_0(raw.ctypes.data, n, _p(out))
    return out


def f16_to_f32(h: int) -> float:
    return float(lib().orc_f16_to_f32(ctypes.c_uint16(h)))


def f32_to_f16(f: float) -> int:
    return int(lib().orc_f32_to_f16(ctypes.c_float(f)))


# ---- logit rules (each returns a copy of the row with the rule applied) ----------------------

def suppress_blank(row, eot):
    r = f32(row).copy()
    lib().orc_suppress_blank(_p(r), r.size, eot)
    return r


def apply_suppress(row, ids):
    r, i = f32(row).copy(), i32(list(ids))
    lib().orc_apply_suppress(_p(r), _p(i, _i32p), i.size, r.size)
    return r


def ngram_block(row, generated, n):
    r, g = f32(row).copy(), i32(list(generated) or [0])
    lib().orc_ngram_block(_p(r), _p(g, _i32p), len(generated), n, r.size)
    return r


def timestamp_rules(row, generated, ts_begin, eot, first_step=False):
    r, g = f32(row).copy(), i32(list(generated) or [0])
    lib().orc_timestamp_rules(_p(r), _p(g, _i32p), len(generated), ts_begin, eot, r.size, int(first_step))
    return r


def needs_fallback(compression_ratio, avg_logprob, no_speech_prob) -> bool:
    return bool(lib().orc_needs_fallback(compression_ratio, avg_logprob, no_speech_prob))


def sample_u(row, temperature, u):
    """(chosen index, the row after the call: the reference overwrites it with exp weights)"""
    r = f32(row).copy()
    k = lib().orc_sample_u(_p(r), r.size, ctypes.c_float(temperature), ctypes.c_double(u))
    return int(k), r


def log_softmax_at(row, index) -> float:
    r = f32(row)
    return float(lib().orc_log_softmax_at(_p(r), r.size, int(index)))


def splitmix64(seed, n):
    st = ctypes.c_uint64(seed)
    return [int(lib().orc_splitmix64_next(ctypes.byref(st))) for _ in range(n)]


def rng_uniform(seed, n):
    st = ctypes.c_uint64(seed)
    return [float(lib().orc_rng_uniform(ctypes.byref(st))) for _ in range(n)]


def fallback_pick(results):
    """results: six dicts (compression_ratio, avg_logprob, no_speech_prob) decoded at 0, 0.2 .. 1.0.
    Returns (index decodeWithFallback returns, number of decodes it runs)."""
    arr = (OrcResult * 6)()
    for i, r in enumerate(results):
        arr[i].n_tokens = 1
        arr[i].tokens[0] = i
        arr[i].compression_ratio = r["compression_ratio"]
        arr[i].avg_logprob = r["avg_logprob"]
        arr[i].no_speech_prob = r["no_speech_prob"]
        arr[i].temperature = 0.2 * i
    used = ctypes.c_int(0)
    k = lib().orc_fallback_pick(arr, ctypes.byref(used))
    return int(k), int(used.value)


class TableSource:
    """Logits source for the decode drivers from a function of each hypothesis's generated tokens:
    rows(tuple_of_generated_tokens) -> logits row; first_row is the prompt's first-position row."""

    def __init__(self, n_vocab, rows, first_row=None):
        self.V, self.rows = n_vocab, rows
        self.first = f32(first_row if first_row is not None else np.zeros(n_vocab))
        self.hist = [()]
        self.calls = []

        def prefill(ctx, first, last):
            self.hist = [()]
            ctypes.memmove(first, self.first.ctypes.data, 4 * self.V)
            r = f32(self.rows(()))
            ctypes.memmove(last, r.ctypes.data, 4 * self.V)
            return 0

        def step(ctx, b, tok, out):
            self.hist[b] = self.hist[b] + (int(tok),)
            self.calls.append((b, self.hist[b]))
            r = f32(self.rows(self.hist[b]))
            ctypes.memmove(out, r.ctypes.data, 4 * self.V)
            return 0

        def rearrange(ctx, src, saved, beam):
            old = list(self.hist) + [()] * (beam - len(self.hist))
            new = [old[src[b]] for b in range(saved)]
            new += [new[0]] * (beam - saved)
            self.hist = new
            return 0

        self._cb = (_PREFILL(prefill), _STEP(step), _REARRANGE(rearrange))
        self.ops = OrcOps(None, *self._cb)


def greedy_drive(src, eot, max_tokens, suppress=(), no_speech=-1, temperature=0.0, ts_begin=-1, seed=0):
    s = i32(list(suppress) or [0])
    r = OrcResult()
    rc = lib().orc_greedy_drive(ctypes.byref(src.ops), src.V, eot, max_tokens, _p(s, _i32p), len(suppress), no_speech,
                                ctypes.c_float(temperature), ts_begin, ctypes.c_uint64(seed), ctypes.byref(r))
    if rc:
        raise ValueError(f"orc_greedy_drive failed ({rc})")
    return r.as_dict()


def beam_drive(src, eot, max_tokens, beam, suppress=(), no_speech=-1, ts_begin=-1):
    s = i32(list(suppress) or [0])
    r = OrcResult()
    rc = lib().orc_beam_drive(ctypes.byref(src.ops), src.V, eot, max_tokens, _p(s, _i32p), len(suppress), no_speech,
                              ts_begin, beam, ctypes.byref(r), None)
    if rc:
        raise ValueError(f"orc_beam_drive failed ({rc})")
    return r.as_dict()


# ---- model ---------------------------------------------------------------------------------

def conv1d(w, bias, stride, pad, x):
    """Conv1d.forward (w [out][in][k], x [in][len]) -> [out][out_len]."""
    w, x = f32(w), f32(x)
    out_ch, in_ch, k = w.shape
    n = x.shape[1]
    out = np.empty((out_ch, (n + 2 * pad - k) // stride + 1), np.float32)
    b = f32(bias) if bias is not None else None
    lib().orc_conv1d(_p(w), _p(b) if b is not None else None, out_ch, in_ch, k, stride, pad, _p(x), n, _p(out))
    return out


class Encoder:
    """Oracle audio encoder (WhisperEncoder) from a GGML tensor table."""

    def __init__(self, edims, tensors):
        self.edims = edims
        self._keep = []
        arr = (OrcTensor * len(tensors))()
        for i, t in enumerate(tensors):
            raw = np.ascontiguousarray(t.raw())
            nm = t.name.encode()
            self._keep += [raw, nm]
            arr[i].name = nm
            arr[i].type = t.ggml_type
            arr[i].n_dims = len(t.ne)
            for j, v in enumerate(t.ne):
                arr[i].ne[j] = int(v)
            arr[i].data = raw.ctypes.data
        self._dims = OrcEncDims(edims.n_mels, edims.n_audio_ctx, edims.n_audio_state, edims.n_audio_head,
                                edims.n_audio_layer)
        err = ctypes.create_string_buffer(256)
        self._h = lib().orc_encoder_create(ctypes.byref(self._dims), arr, len(tensors), err, 256)
        if not self._h:
            raise RuntimeError(err.value.decode())

    def forward(self, mel) -> np.ndarray:
        m = f32(mel)
        out = np.empty((self.edims.n_audio_ctx, self.edims.n_audio_state), np.float32)
        lib().orc_encoder_forward(self._h, _p(m), _p(out))
        return out

    def close(self):
        if self._h:
            lib().orc_encoder_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Model:
    """Oracle decoder built from a GGML tensor table (list of whisper4j_amd.synth.GgmlTensor)."""

    def __init__(self, dims, tensors):
        self.dims = dims
        self._keep = []
        arr = (OrcTensor * len(tensors))()
        for i, t in enumerate(tensors):
            raw = np.ascontiguousarray(t.raw())
            nm = t.name.encode()
            self._keep += [raw, nm]
            arr[i].name = nm
            arr[i].type = t.ggml_type
            arr[i].n_dims = len(t.ne)
            for j, v in enumerate(t.ne):
                arr[i].ne[j] = int(v)
            arr[i].data = raw.ctypes.data
        self._dims = OrcDims(dims.n_vocab, dims.n_text_ctx, dims.n_text_state, dims.n_text_head, dims.n_text_layer,
                             dims.n_audio_ctx)
        err = ctypes.create_string_buffer(512)
        self.h = lib().orc_model_create(ctypes.byref(self._dims), arr, len(tensors), err, 512)
        self._keep = None  # the oracle copies (dequantizes) everything it needs
        if not self.h:
            raise ValueError(err.value.decode())

    def close(self):
        if self.h:
            lib().orc_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_logit_bias(self, bias):
        """Fixed bias [n_vocab] added to every logits row (None: off)."""
        self._bias = None if bias is None else f32(bias)
        lib().orc_model_set_logit_bias(self.h, _p(self._bias))

    def new_cache(self):
        return Cache(self)

    def forward(self, tokens, xa, cache=None) -> np.ndarray:
        t = i32(tokens)
        xa = f32(xa)
        out = np.empty((t.size, self.dims.n_vocab), dtype=np.float32)
        rc = lib().orc_forward(self.h, _p(t, _i32p), t.size, _p(xa), cache.h if cache is not None else None, _p(out))
        if rc:
            raise ValueError(f"orc_forward failed ({rc})")
        return out

    def forced(self, xa, prompt, forced, want_logits=False):
        p, f, xa = i32(prompt), i32(forced), f32(xa)
        n = f.size + 1
        am = np.empty(n, np.int32)
        mx, sec, lse = (np.empty(n, np.float32) for _ in range(3))
        lg = np.empty((n, self.dims.n_vocab), np.float32) if want_logits else None
        rc = lib().orc_forced(self.h, _p(xa), _p(p, _i32p), p.size, _p(f, _i32p), f.size, _p(am, _i32p), _p(mx),
                              _p(sec), _p(lse), _p(lg))
        if rc:
            raise ValueError(f"orc_forced failed ({rc})")
        return {"argmax": am, "max": mx, "second": sec, "lse": lse, "logits": lg}

    def decode(self, xa, prompt, eot, max_tokens, suppress=(), no_speech=-1, temperature=0.0, ts_begin=-1, seed=0):
        p, s, xa = i32(prompt), i32(list(suppress)), f32(xa)
        r = OrcResult()
        rc = lib().orc_decode(self.h, _p(xa), _p(p, _i32p), p.size, eot, max_tokens, _p(s, _i32p), s.size, no_speech,
                              ctypes.c_float(temperature), ts_begin, ctypes.c_uint64(seed), ctypes.byref(r))
        if rc:
            raise ValueError(f"orc_decode failed ({rc})")
        return r.as_dict()

    def decode_beam(self, xa, prompt, eot, max_tokens, suppress=(), no_speech=-1, ts_begin=-1, beam=5):
        p, s, xa = i32(prompt), i32(list(suppress)), f32(xa)
        r = OrcResult()
        rc = lib().orc_decode_beam(self.h, _p(xa), _p(p, _i32p), p.size, eot, max_tokens, _p(s, _i32p), s.size,
                                   no_speech, ts_begin, beam, ctypes.byref(r))
        if rc:
            raise ValueError(f"orc_decode_beam failed ({rc})")
        return r.as_dict()

    def decode_beam_gaps(self, xa, prompt, eot, max_tokens, suppress=(), no_speech=-1, ts_begin=-1, beam=5):
        """decode_beam plus its decision gaps: gaps[i] (search step i) = score of the last hypothesis kept
        minus the first non-end candidate left out, gaps[0] = the final pick's margin."""
        p, s, xa = i32(prompt), i32(list(suppress)), f32(xa)
        r = OrcResult()
        g = np.empty(max_tokens, np.float64)
        rc = lib().orc_decode_beam_gaps(self.h, _p(xa), _p(p, _i32p), p.size, eot, max_tokens, _p(s, _i32p), s.size,
                                        no_speech, ts_begin, beam, ctypes.byref(r),
                                        g.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
        if rc:
            raise ValueError(f"orc_decode_beam_gaps failed ({rc})")
        return r.as_dict(), g

    def decode_with_fallback(self, xa, prompt, eot, max_tokens, suppress=(), no_speech=-1, ts_begin=-1, beam=1,
                             seed=0):
        p, s, xa = i32(prompt), i32(list(suppress)), f32(xa)
        r = OrcResult()
        rc = lib().orc_decode_with_fallback(self.h, _p(xa), _p(p, _i32p), p.size, eot, max_tokens, _p(s, _i32p),
                                            s.size, no_speech, ts_begin, beam, ctypes.c_uint64(seed), ctypes.byref(r))
        if rc:
            raise ValueError(f"orc_decode_with_fallback failed ({rc})")
        return r.as_dict()


class Cache:
    def __init__(self, model: Model):
        self.h = lib().orc_cache_create(model.h)

    def __len__(self):
        return int(lib().orc_cache_len(self.h))

    def close(self):
        if self.h:
            lib().orc_cache_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
