import importlib.util
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "tests"))


def load_package():
    """Import the package directory prime-tts_amd/ (its name is not a Python identifier)."""
    if "prime_tts_amd" in sys.modules:
        return sys.modules["prime_tts_amd"]
    init = ROOT / "prime-tts_amd" / "__init__.py"
    spec = importlib.util.spec_from_file_location("prime_tts_amd", init,
                                                  submodule_search_locations=[str(init.parent)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["prime_tts_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def pkg():
    return load_package()


class KnobEnv:
    """monkeypatch's setenv / delenv for the library's tuning knobs (PTK_CONV_*, PTK_TAIL_*,
    PTD_WINDOW_*), which the library reads once per process: each change is followed by
    ptd_debug_reload_env, so the next call sees it."""

    def __init__(self, mp):
        self._mp = mp

    @staticmethod
    def reload():
        load_package().load().ptd_debug_reload_env()

    def setenv(self, name, value):
        self._mp.setenv(name, value)
        self.reload()

    def delenv(self, name, raising=True):
        self._mp.delenv(name, raising=raising)
        self.reload()


@pytest.fixture
def knob_env(monkeypatch):
    """Knob changes for one test; the environment is restored and re-read when it ends."""
    yield KnobEnv(monkeypatch)
    monkeypatch.undo()
    KnobEnv.reload()
