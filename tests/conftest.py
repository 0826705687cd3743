import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "mormot2-qwen-tts_amd"), os.path.join(ROOT, "oracle"),
          os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


@pytest.fixture(scope="session")
def q3h():
    import q3h as m
    m.lib()
    return m


@pytest.fixture(scope="session")
def q3o():
    import q3o as m
    m.lib()
    return m


@pytest.fixture(scope="session")
def synth():
    import synth as m
    return m


@pytest.fixture(scope="session")
def device(q3h):
    if not q3h.available():
        pytest.fail("no gfx950 device: the gpu tests need the HIP library on an MI355X")
    d = q3h.Device(0)
    yield d
    d.close()
