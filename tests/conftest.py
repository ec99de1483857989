import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def load_package():
    """The package directory intel-phi-apl_amd/ under the importable name q8rt."""
    if "q8rt" in sys.modules:
        return sys.modules["q8rt"]
    spec = importlib.util.spec_from_file_location("q8rt", os.path.join(ROOT, "intel-phi-apl_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["q8rt"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def q8rt():
    return load_package()


@pytest.fixture(scope="session")
def oracle():
    from oracle_ffi import Oracle

    return Oracle()


@pytest.fixture(scope="session")
def reference():
    from oracle_ffi import reference_or_none

    return reference_or_none()


@pytest.fixture(scope="session")
def rt(q8rt):
    """One GPU runtime for the whole GPU session; a GPU test fails (never skips) without it."""
    r = q8rt.Runtime()
    yield r
    r.close()
