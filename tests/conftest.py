"""Shared fixtures.

`gpu`-marked tests need an MI355X and the built library; everything else
runs on the CPU (oracle pins, host logic, ABI/export checks).
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "qora-llm-4b_amd"


def _load(name: str, path: Path):
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def load_mixer():
    return _load("qora_mixer", PKG / "qora_mixer.py")


def load_workloads():
    return _load("qora_workloads", PKG / "workloads.py")


def load_oracle():
    return _load("qora_oracle_py", ROOT / "oracle" / "oracle.py")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def mixer():
    return load_mixer()


@pytest.fixture(scope="session")
def oracle():
    return load_oracle()


@pytest.fixture(scope="session")
def workloads():
    return load_workloads()


@pytest.fixture(scope="session")
def ctx(mixer):
    """A mixer context on device 0 (GPU tests only)."""
    c = mixer.Context(0)
    yield c
    c.close()
