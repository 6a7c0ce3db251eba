"""CPU: the .qor4b parser (qora-llm-4b_amd/host/qor4b_file.hpp) against files
written field for field as save_model does (save.rs:135-240), and its load
errors (save.rs:247-260,127); the checks are in tests/cpp/qor4b_file_test.cpp."""
from __future__ import annotations

import subprocess

from conftest import PKG


def test_qor4b_parser():
    exe = PKG / "lib" / "qor4b_file_test"
    assert exe.exists(), "build with qora-llm-4b_amd/build.py"
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all checks passed" in r.stdout
