import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture
def tuning_env(monkeypatch):
    """Sets LMX_* kernel-choice overrides for one test.  The library reads
    them once, so every change is followed by lmx.tuning_reload(), and the
    environment is restored and re-read after the test."""
    import llmoxide_amd as lmx

    def setenv(name, value):
        monkeypatch.setenv(name, value)
        lmx.tuning_reload()
    yield setenv
    monkeypatch.undo()
    lmx.tuning_reload()
