"""CPU: the GQA prefill attention's row-block order (qm_gqa_plan.h, used by
qm_gqa_prefill): each order hands out every block once, the queue model
matches hand-worked and brute-force cases, and the automatic choice takes the
packed order only where longest first is at least 5% behind it (8192
tokens); the checks are in tests/cpp/gqa_plan_test.cpp."""
from __future__ import annotations

import subprocess

from conftest import PKG


def test_gqa_prefill_block_order_plan():
    exe = PKG / "lib" / "gqa_plan_test"
    assert exe.exists(), "build with qora-llm-4b_amd/build.py"
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all checks passed" in r.stdout
