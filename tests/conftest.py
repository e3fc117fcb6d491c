import importlib.util
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(REPO, "flash-infer-bench-starter-kit_amd")
ORACLE_DIR = os.path.join(REPO, "oracle")
GOLDEN_DIR = os.path.join(REPO, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


def load_module(name: str, path: str):
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def pkg(name: str):
    """Import a module of the (hyphen-named) package directory by file path."""
    return load_module(f"moe_mi355_{name}", os.path.join(PKG_DIR, f"{name}.py"))


def oracle():
    return load_module("moe_oracle", os.path.join(ORACLE_DIR, "moe_oracle.py"))


@pytest.fixture(scope="session")
def orc():
    return oracle()


@pytest.fixture(scope="session")
def kmod():
    return pkg("kernel")


@pytest.fixture(scope="session")
def wl():
    return pkg("workloads")
