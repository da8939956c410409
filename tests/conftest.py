import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _reload_combs_options():
    """The library reads its COMBS_* tuning variables once; re-read them after
    a test changes one (only if the library is already loaded)."""
    from combsengine_amd import _lib as L
    if L._lib is not None:
        L.reload_options()


@pytest.fixture
def monkeypatch():
    """pytest's monkeypatch, re-reading the library's options whenever a
    COMBS_* variable is set and after the test's changes are undone."""
    from _pytest.monkeypatch import MonkeyPatch
    mp = MonkeyPatch()
    setenv = mp.setenv

    def _setenv(name, value, prepend=None):
        setenv(name, value, prepend)
        if name.startswith("COMBS_"):
            _reload_combs_options()

    mp.setenv = _setenv
    delenv = mp.delenv

    def _delenv(name, raising=True):
        delenv(name, raising)
        if name.startswith("COMBS_"):
            _reload_combs_options()

    mp.delenv = _delenv
    yield mp
    mp.undo()
    _reload_combs_options()
