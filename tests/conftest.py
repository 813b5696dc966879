import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def hip():
    """(device, stream) of the hip backend on GPU 0."""
    import scrapgpulibrary_amd as sg

    dev = sg.Device(0)
    st = dev.stream()
    yield dev, st
    st.free()
