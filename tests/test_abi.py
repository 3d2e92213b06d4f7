"""C ABI checks that need no GPU: the library loads, exports every declared symbol, parses GGML
files with the reference loader's format rules, and reports errors as codes plus a message."""

import os
import re
import struct

import numpy as np
import pytest

from whisper4j_amd import _lib, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SMALL = synth.Dims(n_vocab=300, n_text_ctx=16, n_text_state=64, n_text_head=1, n_text_layer=1, n_audio_ctx=20)


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "w4h.h")).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(w4h_[a-z0-9_]+)\s*\(", text, re.M)))


def test_exports_every_declared_symbol(w4h):
    decl = declared_symbols()
    assert len(decl) >= 25
    assert sorted(_lib.EXPORTS) == decl
    lib = w4h.lib()
    for name in decl:
        assert getattr(lib, name) is not None


def test_device_count_is_not_an_error(w4h):
    assert w4h.device_count() >= 0


@pytest.fixture()
def ggml_file(tmp_path):
    T = synth.make_decoder(SMALL, seed=3)
    path = str(tmp_path / "ggml-small.bin")
    synth.write_ggml(path, SMALL, T)
    return path, T


def test_ggml_inspect_and_read(w4h, ggml_file):
    import ctypes

    path, T = ggml_file
    d = _lib.Dims()
    n = ctypes.c_int32()
    nbytes = ctypes.c_int64()
    _lib.check(w4h.lib().w4h_ggml_inspect(path.encode(), ctypes.byref(d), ctypes.byref(n), ctypes.byref(nbytes)))
    assert (d.n_vocab, d.n_text_ctx, d.n_text_state, d.n_text_head, d.n_text_layer, d.n_audio_ctx) == (
        300, 16, 64, 1, 1, 20)
    assert n.value == len(T)
    assert nbytes.value == sum(t.raw().nbytes for t in T)
    for t in (T[0], T[5], T[-1]):
        ty, nd = ctypes.c_int32(), ctypes.c_int32()
        ne = (ctypes.c_int64 * 4)()
        buf = np.empty(t.raw().nbytes, np.uint8)
        _lib.check(w4h.lib().w4h_ggml_read_tensor(path.encode(), t.name.encode(), ctypes.byref(ty), ctypes.byref(nd),
                                                 ne, buf.ctypes.data, buf.nbytes))
        assert ty.value == t.ggml_type and nd.value == len(t.ne)
        assert tuple(ne[: nd.value]) == tuple(t.ne)
        np.testing.assert_array_equal(buf, t.raw())


def _expect(w4h, code, fn, *args):
    rc = fn(*args)
    assert rc == code, (rc, w4h.lib().w4h_last_error())
    assert w4h.lib().w4h_last_error()


def test_ggml_errors(w4h, ggml_file, tmp_path):
    import ctypes

    path, T = ggml_file
    L = w4h.lib()
    d = _lib.Dims()
    n = ctypes.c_int32()
    b = ctypes.c_int64()
    # missing file (IOException in the reference)
    _expect(w4h, _lib.W4H_ERR_IO, L.w4h_ggml_inspect, str(tmp_path / "nope.bin").encode(), ctypes.byref(d),
            ctypes.byref(n), ctypes.byref(b))
    # bad magic (GgmlLoader.java:98-99)
    bad = tmp_path / "bad.bin"
    bad.write_bytes(struct.pack("<i", 0x12345678) + b"\0" * 64)
    _expect(w4h, _lib.W4H_ERR_FORMAT, L.w4h_ggml_inspect, str(bad).encode(), ctypes.byref(d), ctypes.byref(n),
            ctypes.byref(b))
    # truncated tensor data
    raw = open(path, "rb").read()
    trunc = tmp_path / "trunc.bin"
    trunc.write_bytes(raw[: len(raw) - 100])
    _expect(w4h, _lib.W4H_ERR_FORMAT, L.w4h_ggml_inspect, str(trunc).encode(), ctypes.byref(d), ctypes.byref(n),
            ctypes.byref(b))
    # missing tensor name (WeightStore.get, model/WeightStore.java:28-34)
    ty, nd = ctypes.c_int32(), ctypes.c_int32()
    ne = (ctypes.c_int64 * 4)()
    _expect(w4h, _lib.W4H_ERR_NOT_FOUND, L.w4h_ggml_read_tensor, path.encode(), b"decoder.nope", ctypes.byref(ty),
            ctypes.byref(nd), ne, None, 0)


def test_ggml_stops_at_implausible_header(w4h, ggml_file, tmp_path):
    # GgmlLoader.java:153-158: an implausible tensor header ends the tensor list
    import ctypes

    path, T = ggml_file
    junk = tmp_path / "junk.bin"
    junk.write_bytes(open(path, "rb").read() + struct.pack("<iii", 9, 1, 0))
    d, n, b = _lib.Dims(), ctypes.c_int32(), ctypes.c_int64()
    _lib.check(w4h.lib().w4h_ggml_inspect(str(junk).encode(), ctypes.byref(d), ctypes.byref(n), ctypes.byref(b)))
    assert n.value == len(T)


def test_null_and_range_arguments(w4h):
    import ctypes

    L = w4h.lib()
    _expect(w4h, _lib.W4H_ERR_INVALID, L.w4h_model_create, None, None, 0, 0, None)
    _expect(w4h, _lib.W4H_ERR_INVALID, L.w4h_session_create, None, None, None)
    _expect(w4h, _lib.W4H_ERR_INVALID, L.w4h_model_destroy, None)
    _expect(w4h, _lib.W4H_ERR_INVALID, L.w4h_op_linear, None, 1, 8, 32, None, None, 1, None)
    r = ctypes.c_float()
    _expect(w4h, _lib.W4H_ERR_INVALID, L.w4h_compression_ratio, None, -1, ctypes.byref(r))


def test_compression_ratio_matches_oracle(w4h, orc):
    toks = list(range(100, 160)) * 3
    assert w4h.compression_ratio(toks) == pytest.approx(orc.compression_ratio(toks), rel=1e-6)
    assert w4h.compression_ratio([]) == 0.0


def test_no_device_reports_device_error(w4h):
    if w4h.device_count() > 0:
        pytest.skip("a GPU is visible")
    T = synth.make_decoder(SMALL, seed=1)
    with pytest.raises(w4h.W4HError) as e:
        w4h.Model.from_tensors(SMALL, T)
    assert e.value.code == _lib.W4H_ERR_DEVICE
