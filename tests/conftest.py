import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libk44wavec.so on the GPU)")


@pytest.fixture(scope="session")
def wavec():
    from snntome_amd import wavec as wv

    wv.get_lib()  # fails loudly if the library was not built
    return wv


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle

    oracle.lib()
    return oracle


@pytest.fixture
def tuning(wavec):
    """wavec.set_tuning for the duration of one test: every executor tuning switch is back to
    automatic (-1) before and after it."""
    wavec.reset_tuning()
    yield wavec.set_tuning
    wavec.reset_tuning()
