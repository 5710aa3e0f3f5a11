"""Shared fixtures.  GPU tests are marked `gpu`; everything else runs on CPU."""
import importlib.util
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


def load_pkg():
    """Import the product package from fast-llm_amd/ (a hyphenated directory)."""
    if "fast_llm_amd" in sys.modules:
        return sys.modules["fast_llm_amd"]
    spec = importlib.util.spec_from_file_location(
        "fast_llm_amd", os.path.join(ROOT, "fast-llm_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["fast_llm_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def flh():
    return load_pkg()


@pytest.fixture(scope="session")
def orc():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def golden():
    return np.load(os.path.join(ROOT, "tests", "golden", "golden_ref.npz"), allow_pickle=False)


@pytest.fixture(scope="session")
def gpu(flh):
    """Initialised device + stream; fails (never falls back) without a GPU."""
    flh.init(0)
    s = flh.Stream()
    yield s
    s.sync()
    s.close()
