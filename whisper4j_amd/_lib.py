"""ctypes binding of libw4h.so (the C ABI declared in include/w4h.h).

Loading never falls back to anything: a missing or unloadable library raises immediately.
"""

from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libw4h.so")

W4H_OK = 0
W4H_SELECT_MAX_ROWS = 64  # rows of the allocation-free selection's fixed partials array
W4H_ERR_INVALID = -1
W4H_ERR_NOT_FOUND = -2
W4H_ERR_SHAPE = -3
W4H_ERR_FORMAT = -4
W4H_ERR_DEVICE = -5
W4H_ERR_OOM = -6
W4H_ERR_CLOSED = -7
W4H_ERR_CAPACITY = -8
W4H_ERR_TIMEOUT = -9
W4H_ERR_IO = -10
W4H_ERR_CANCELLED = -11
TOPK_MAX = 8

TYPE_F32, TYPE_F16, TYPE_Q8_0 = 0, 1, 8

# Every symbol include/w4h.h declares.
EXPORTS = (
    "w4h_last_error", "w4h_device_count", "w4h_model_create", "w4h_model_load_ggml", "w4h_model_dims",
    "w4h_model_destroy", "w4h_encoder_create", "w4h_encoder_load_ggml", "w4h_encoder_get_dims",
    "w4h_encoder_forward", "w4h_encoder_forward_device", "w4h_encoder_destroy", "w4h_ggml_inspect", "w4h_ggml_read_tensor", "w4h_session_create", "w4h_session_destroy",
    "w4h_session_set_encoder", "w4h_session_set_encoder_device", "w4h_session_reset", "w4h_session_kv_len", "w4h_session_set_suppress",
    "w4h_session_set_probe", "w4h_session_set_logit_bias", "w4h_session_cancel", "w4h_session_step", "w4h_session_run", "w4h_session_reorder", "w4h_session_time_run",
    "w4h_session_trace_run",
    "w4h_decode", "w4h_decode_beam", "w4h_decode_with_fallback", "w4h_compression_ratio", "w4h_op_linear",
    "w4h_op_layernorm", "w4h_op_gelu", "w4h_op_attention", "w4h_op_select", "w4h_op_sample",
    "w4h_op_select_noalloc",
)


class W4HError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class Tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_int32), ("n_dims", ctypes.c_int32),
                ("ne", ctypes.c_int64 * 4), ("data", ctypes.c_void_p)]


class Dims(ctypes.Structure):
    _fields_ = [("n_vocab", ctypes.c_int32), ("n_text_ctx", ctypes.c_int32), ("n_text_state", ctypes.c_int32),
                ("n_text_head", ctypes.c_int32), ("n_text_layer", ctypes.c_int32), ("n_audio_ctx", ctypes.c_int32)]


class EncoderDims(ctypes.Structure):
    _fields_ = [("n_mels", ctypes.c_int32), ("n_audio_ctx", ctypes.c_int32), ("n_audio_state", ctypes.c_int32),
                ("n_audio_head", ctypes.c_int32), ("n_audio_layer", ctypes.c_int32)]


class SessionDesc(ctypes.Structure):
    _fields_ = [("n_rows", ctypes.c_int32), ("n_encoders", ctypes.c_int32), ("max_ctx", ctypes.c_int32)]


class StepOut(ctypes.Structure):
    _fields_ = [("argmax", ctypes.c_int32), ("max_logit", ctypes.c_float), ("logsumexp", ctypes.c_float),
                ("probe_logit", ctypes.c_float), ("raw_logsumexp", ctypes.c_float),
                ("topk_ids", ctypes.c_int32 * TOPK_MAX), ("topk_logits", ctypes.c_float * TOPK_MAX)]


class DecodeOpts(ctypes.Structure):
    _fields_ = [("prompt", ctypes.POINTER(ctypes.c_int32)), ("n_prompt", ctypes.c_int32), ("eot", ctypes.c_int32),
                ("max_tokens", ctypes.c_int32), ("suppress", ctypes.POINTER(ctypes.c_int32)),
                ("n_suppress", ctypes.c_int32), ("no_speech", ctypes.c_int32), ("temperature", ctypes.c_float),
                ("timestamp_begin", ctypes.c_int32), ("beam_size", ctypes.c_int32), ("seed", ctypes.c_uint64)]


class DecodeResult(ctypes.Structure):
    _fields_ = [("n_tokens", ctypes.c_int32), ("tokens", ctypes.c_int32 * 1024), ("avg_logprob", ctypes.c_float),
                ("compression_ratio", ctypes.c_float), ("no_speech_prob", ctypes.c_float),
                ("temperature", ctypes.c_float)]


_lib = None


def lib():
    """Load libw4h.so (raises OSError if it is missing or does not load)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise OSError(f"{LIB_PATH} is not built; run `python -m whisper4j_amd.build` or __graft_entry__.build()")
    L = ctypes.CDLL(LIB_PATH)
    vp, i32, f32p, i32p = ctypes.c_void_p, ctypes.c_int32, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_int32)
    u32p, u16p = ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint16)
    sig = {
        "w4h_last_error": (ctypes.c_char_p, []),
        "w4h_device_count": (i32, [i32p]),
        "w4h_model_create": (i32, [ctypes.POINTER(Dims), ctypes.POINTER(Tensor), i32, i32, ctypes.POINTER(vp)]),
        "w4h_model_load_ggml": (i32, [ctypes.c_char_p, i32, ctypes.POINTER(vp)]),
        "w4h_model_dims": (i32, [vp, ctypes.POINTER(Dims)]),
        "w4h_model_destroy": (i32, [vp]),
        "w4h_encoder_create": (i32, [ctypes.POINTER(EncoderDims), ctypes.POINTER(Tensor), i32, i32, ctypes.POINTER(vp)]),
        "w4h_encoder_load_ggml": (i32, [ctypes.c_char_p, i32, ctypes.POINTER(vp)]),
        "w4h_encoder_get_dims": (i32, [vp, ctypes.POINTER(EncoderDims)]),
        "w4h_encoder_forward": (i32, [vp, f32p, f32p]),
        "w4h_encoder_forward_device": (i32, [vp, vp, vp, vp]),
        "w4h_encoder_destroy": (i32, [vp]),
        "w4h_ggml_inspect": (i32, [ctypes.c_char_p, ctypes.POINTER(Dims), i32p, ctypes.POINTER(ctypes.c_int64)]),
        "w4h_ggml_read_tensor": (i32, [ctypes.c_char_p, ctypes.c_char_p, i32p, i32p, ctypes.c_int64 * 4, vp,
                                       ctypes.c_int64]),
        "w4h_session_create": (i32, [vp, ctypes.POINTER(SessionDesc), ctypes.POINTER(vp)]),
        "w4h_session_destroy": (i32, [vp]),
        "w4h_session_set_encoder": (i32, [vp, i32, f32p]),
        "w4h_session_set_encoder_device": (i32, [vp, i32, vp]),
        "w4h_session_reset": (i32, [vp, i32]),
        "w4h_session_kv_len": (i32, [vp, i32p]),
        "w4h_session_set_suppress": (i32, [vp, i32p, i32]),
        "w4h_session_set_probe": (i32, [vp, i32]),
        "w4h_session_set_logit_bias": (i32, [vp, f32p]),
        "w4h_session_cancel": (i32, [vp, i32]),
        "w4h_session_step": (i32, [vp, i32p, u32p, i32, ctypes.POINTER(StepOut), f32p]),
        "w4h_session_run": (i32, [vp, i32p, i32p, i32, i32, ctypes.POINTER(StepOut)]),
        "w4h_session_reorder": (i32, [vp, i32p]),
        "w4h_session_time_run": (i32, [vp, i32p, i32p, i32, i32, f32p, ctypes.POINTER(StepOut)]),
        "w4h_session_trace_run": (i32, [vp, i32p, i32p, i32, ctypes.POINTER(ctypes.c_uint64), ctypes.c_int64, i32p]),
        "w4h_decode": (i32, [vp, ctypes.POINTER(DecodeOpts), ctypes.POINTER(DecodeResult)]),
        "w4h_decode_beam": (i32, [vp, ctypes.POINTER(DecodeOpts), ctypes.POINTER(DecodeResult)]),
        "w4h_decode_with_fallback": (i32, [vp, ctypes.POINTER(DecodeOpts), ctypes.POINTER(DecodeResult)]),
        "w4h_compression_ratio": (i32, [i32p, i32, f32p]),
        "w4h_op_linear": (i32, [vp, i32, i32, i32, f32p, f32p, i32, f32p]),
        "w4h_op_layernorm": (i32, [f32p, i32, i32, f32p, f32p, f32p]),
        "w4h_op_gelu": (i32, [f32p, i32, f32p]),
        "w4h_op_attention": (i32, [f32p, u16p, u16p, i32, i32, ctypes.c_float, f32p]),
        "w4h_op_select": (i32, [f32p, i32, i32, u32p, i32, ctypes.POINTER(StepOut)]),
        "w4h_op_sample": (i32, [f32p, i32, u32p, i32p, i32, i32, i32, ctypes.c_float, ctypes.c_uint64, i32p,
                                ctypes.POINTER(ctypes.c_double)]),
        "w4h_op_select_noalloc": (i32, [vp, i32, i32, vp, i32, vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != W4H_OK:
        msg = lib().w4h_last_error()
        raise W4HError(rc, msg.decode() if msg else "")


def device_count() -> int:
    n = ctypes.c_int32(0)
    check(lib().w4h_device_count(ctypes.byref(n)))
    return n.value
