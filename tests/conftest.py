"""pytest configuration: the `gpu` marker, the repo root on sys.path, and a build-if-missing hook
for the native libraries (tests load what is built and only build when nothing is)."""
import importlib.util
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
if str(ROOT / "tests") not in sys.path:
    sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _ensure_built():
    spec = importlib.util.spec_from_file_location("qe_build", ROOT / "qengine_amd" / "_build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    if not mod.built():
        mod.build()


@pytest.fixture(scope="session")
def native():
    """The built torch extension module qengine_amd._C (builds once if nothing is built)."""
    _ensure_built()
    import qengine_amd
    return qengine_amd._C


@pytest.fixture(scope="session")
def capi():
    """ctypes binding of libqe_attn.so (builds once if nothing is built)."""
    _ensure_built()
    from qengine_amd import capi as c
    c.load()
    return c
