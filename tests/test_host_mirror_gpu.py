"""GPU: the C++ mirror of the reference layer-forwards (qor4b_mixer.hpp),
driven through prefill -> decode flows with state carried over, checked
against the CPU oracle inside tests/cpp/host_mirror_test.cpp."""
from __future__ import annotations

import subprocess

import pytest

from conftest import PKG

pytestmark = pytest.mark.gpu


def test_host_mirror_flows():
    exe = PKG / "lib" / "host_mirror_test"
    assert exe.exists(), "build with qora-llm-4b_amd/build.py"
    print("case: C++ mirror prefill->decode flows", flush=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
