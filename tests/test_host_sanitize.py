"""The GGML file parser under AddressSanitizer and UndefinedBehaviorSanitizer (host code, no GPU).

The parser reads untrusted files, so it is built with -fsanitize=address,undefined (and errors fatal)
together with tests/host/ggml_sanitize_driver.cpp, and run over a valid decoder file written from a
tensor table plus damaged copies of it: every prefix length across the header and the first tensors,
bytes overwritten with random values at seeded offsets, and implausible dimensions.  Each file must
end in a return code; any memory error or undefined behaviour aborts the run.
"""

import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

from whisper4j_amd import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SMALL = synth.Dims(n_vocab=120, n_text_ctx=8, n_text_state=64, n_text_head=1, n_text_layer=1, n_audio_ctx=10)


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("no g++ on this host")
    out = str(tmp_path_factory.mktemp("san") / "ggml_san")
    cmd = [cxx, "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-fno-omit-frame-pointer", "-I", os.path.join(ROOT, "include"),
           os.path.join(ROOT, "whisper4j_amd", "csrc", "w4h_ggml.cpp"),
           os.path.join(ROOT, "tests", "host", "ggml_sanitize_driver.cpp"), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return out


def test_ggml_parser_sanitized(driver, tmp_path):
    files = []
    for wtype in ("f16", "q8_0"):
        T = synth.make_decoder(SMALL, seed=7, wtype=wtype)
        path = str(tmp_path / f"good-{wtype}.bin")
        synth.write_ggml(path, SMALL, T, ftype=1)
        names = "\n".join(t.name for t in T) + "\ndecoder.nope\n"
        raw = open(path, "rb").read()
        variants = {"good": raw}
        for cut in list(range(0, 200, 3)) + list(range(200, len(raw), max(1, len(raw) // 60))):
            variants[f"cut{cut}"] = raw[:cut]
        rng = np.random.default_rng(11)
        for k in range(60):
            b = bytearray(raw)
            for off in rng.integers(0, min(len(b), 400), 4):
                b[int(off)] = int(rng.integers(0, 256))
            variants[f"flip{k}"] = bytes(b)
        # implausible first tensor header: huge dims, negative name length, unknown type
        head = 4 + 11 * 4 + 8 + 4
        for k, (nd, nl, ty, ne0) in enumerate([(2, 30, 1, 2 ** 31 - 1), (4, -5, 1, 8), (2, 30, 77, 8), (9, 30, 1, 8),
                                                (2, 10 ** 6, 1, 8), (2, 30, 8, 33)]):
            b = bytearray(raw)
            struct.pack_into("<iiii", b, head, nd, nl, ty, ne0)
            variants[f"hdr{k}"] = bytes(b)
        for name, data in variants.items():
            p = str(tmp_path / f"{wtype}-{name}.bin")
            open(p, "wb").write(data)
            open(p + ".names", "w").write(names)
            files.append(p)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1", UBSAN_OPTIONS="halt_on_error=1")
    r = subprocess.run([driver] + files, capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, (r.stdout[-500:], r.stderr[-3000:])
    words = r.stdout.replace(",", " ").split()
    parsed, refused = int(words[1]), int(words[3])
    assert parsed >= 2 and refused >= 20
