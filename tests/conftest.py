import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as o
    o.build()
    return o


@pytest.fixture(scope="session")
def golden():
    import numpy as np
    path = os.path.join(ROOT, "tests", "golden", "golden.npz")
    with np.load(path, allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


def load_tmc():
    """Import the backend package (its directory name is not a Python identifier)."""
    import importlib.util
    name = "aicompiler_test_amd"
    if name in sys.modules:
        return sys.modules[name]
    pkg_dir = os.path.join(ROOT, "aicompiler-test_amd")
    spec = importlib.util.spec_from_file_location(
        name, os.path.join(pkg_dir, "__init__.py"), submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def tmc():
    return load_tmc()


@pytest.fixture(scope="session")
def host(tmc):
    """The C++ host layer module (_tmc_host)."""
    return tmc.host()


@pytest.fixture(autouse=True)
def _announce(request):
    # Name the case before any GPU work so a crash log identifies it.
    if request.node.get_closest_marker("gpu"):
        print(f"\n[gpu-case] {request.node.nodeid}", flush=True)
    yield
