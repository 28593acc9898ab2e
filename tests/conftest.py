import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libvbhip.so")


def pytest_collection_modifyitems(config, items):
    # GPU tests print the case before they run so a hang or fault names it.
    pass


@pytest.fixture(autouse=True)
def _announce(request):
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[case] {request.node.nodeid}", flush=True)
    yield


@pytest.fixture
def knob(monkeypatch):
    """Set a launch-tuning environment override for one test: the library
    reads the overrides once, so each change is followed by
    vb_tuning_reload(), and the original environment is reloaded after the
    test."""
    from vibeblade_amd import _lib
    lib = _lib.load()

    def set_knob(name, value):
        monkeypatch.setenv(name, value)
        lib.vb_tuning_reload()

    yield set_knob
    monkeypatch.undo()
    lib.vb_tuning_reload()
