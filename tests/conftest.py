"""Shared test setup: markers, import paths, the oracle / reference / product handles."""
import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def load_package():
    """Import rich-triplet-cpp_amd/ as `rich_triplet_cpp_amd`."""
    name = "rich_triplet_cpp_amd"
    if name in sys.modules:
        return sys.modules[name]
    path = os.path.join(ROOT, "rich-triplet-cpp_amd", "__init__.py")
    spec = importlib.util.spec_from_file_location(name, path,
                                                  submodule_search_locations=[os.path.dirname(path)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def orc():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle import Reference, reference_available
    if not reference_available():
        pytest.skip("oracle/_ref/libref_oracle.so not built (reference tree absent)")
    return Reference()


@pytest.fixture(scope="session")
def rt():
    """The product binding; on a GPU box it must load and find a gfx950."""
    pkg = load_package()
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    pkg.rt_hip.init(0)
    return pkg.rt_hip
