import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path through the C ABI)")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def w4h():
    import whisper4j_amd

    whisper4j_amd.lib()
    return whisper4j_amd


@pytest.fixture(scope="session")
def gpu(w4h):
    if w4h.device_count() < 1:
        pytest.fail("no HIP device visible to libw4h.so")
    return w4h
