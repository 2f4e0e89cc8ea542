import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP sampler)")
    config.addinivalue_line("markers", "slow: exhaustive CPU checks (tens of seconds)")


def load_pkg():
    """Import the package directory nim.llm_amd/ as module `nimllm_amd`."""
    import importlib.util

    name = "nimllm_amd"
    if name in sys.modules:
        return sys.modules[name]
    pdir = os.path.join(ROOT, "nim.llm_amd")
    spec = importlib.util.spec_from_file_location(name, os.path.join(pdir, "__init__.py"),
                                                  submodule_search_locations=[pdir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def pkg():
    return load_pkg()
