"""Shared fixtures. `gpu` tests need an MI355X; everything else runs on CPU."""
import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PKG_DIR = os.path.join(ROOT, "saphira-llm_amd")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 (MI355X) device")


def load_package():
    """The bindings module of saphira-llm_amd/ (hyphenated directory, loaded by path)."""
    name = "saphira_llm_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(PKG_DIR, "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def amd():
    mod = load_package()
    # SLLM_TEST_LIB: run the tests against another build of the library's C
    # sources (the sanitizer build of tests/fakehip, tests/test_sanitizers.py)
    if os.environ.get("SLLM_TEST_LIB"):
        mod.LIB_PATH = os.environ["SLLM_TEST_LIB"]
    return mod


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    return oracle


@pytest.fixture(scope="session")
def dev(amd):
    """The opened gfx950 device. Fails (does not skip) when it cannot open."""
    d = amd.Device(0)
    print(f"\n[device] {d.name} cu={d.cu} hbm={d.hbm / 2**30:.1f} GiB", flush=True)
    return d
