"""Shared fixtures: the HIP package (loaded by path: its directory name has a hyphen), the CPU oracle, and the
`gpu` marker. GPU tests need a visible device AND the built library; without a device they are skipped."""
import importlib.util
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "qwen27-engine_amd")
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def load_package():
    name = "qwen27_engine_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def q27():
    return load_package()


@pytest.fixture(scope="session")
def oracle():
    from oracle import q27_oracle

    q27_oracle.lib()
    return q27_oracle


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")


def bits(a):
    """Raw bit pattern of a numpy array (for bit-exact comparisons of float outputs)."""
    a = np.ascontiguousarray(a)
    return a.view(np.uint8)


def assert_bits_equal(got, want, what):
    got = np.ascontiguousarray(got)
    want = np.ascontiguousarray(want)
    assert got.shape == want.shape, f"{what}: shape {got.shape} vs {want.shape}"
    if got.dtype.kind == "f":
        gi, wi = got.view(np.int32 if got.itemsize == 4 else np.int16), want.view(np.int32 if want.itemsize == 4 else np.int16)
    else:
        gi, wi = got, want
    bad = np.flatnonzero(gi.reshape(-1) != wi.reshape(-1))
    assert bad.size == 0, (f"{what}: {bad.size} of {got.size} differ; first at {bad[0]}: "
                           f"{got.reshape(-1)[bad[0]]!r} vs {want.reshape(-1)[bad[0]]!r}")
