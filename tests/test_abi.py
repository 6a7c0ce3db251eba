"""CPU-side checks of the C ABI: exports, code objects, argument validation.

No kernel is launched here.  Argument checks run before any device work, so
they are exercised on the CPU host (where qm_create reports no device).
"""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

from conftest import ROOT, load_mixer, load_oracle

M = load_mixer()
HEADER = ROOT / "include" / "qora_mixer.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_mixer_entries():
    syms = declared_symbols()
    for s in ["qm_create", "qm_destroy", "qm_deltanet_decode", "qm_deltanet_prefill",
              "qm_gqa_decode", "qm_gqa_prefill", "qm_q4_gemv", "qm_status_string", "qm_last_error"]:
        assert s in syms


def test_library_exports_every_declared_symbol():
    lib = M.load_library()
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    # and the binding declares every one of them
    assert set(declared_symbols()) <= set(M._SIGNATURES)


def test_code_objects_are_gfx950_bundles():
    for name in ["qm_dn_decode", "qm_gqa_decode", "qm_util", "qm_dn_prefill", "qm_gqa_prefill", "qm_q4_proj",
                 "qm_q4_vocab", "qm_sample"]:
        p = M.LIB_DIR / f"{name}.hsaco"
        assert p.exists(), p
        data = p.read_bytes()
        assert data.startswith(b"__CLANG_OFFLOAD_BUNDLE__") or data[:4] == b"\x7fELF"
        assert b"gfx950" in data


def test_status_strings():
    lib = M.load_library()
    for code in range(10):
        assert lib.qm_status_string(code).decode() != "unknown status"
    assert lib.qm_status_string(99).decode() == "unknown status"


def test_create_rejects_other_shapes_before_touching_a_device():
    lib = M.load_library()
    cfg = M.default_config()
    cfg.attn_head_dim = 128
    h = C.c_void_p(0)
    st = lib.qm_create(C.byref(h), C.byref(cfg), None, 0)
    assert st == 4 and not h.value                            # QM_ERR_SHAPE
    assert "4B mixer" in lib.qm_last_error(None).decode()


def test_null_context_and_null_out():
    lib = M.load_library()
    assert lib.qm_create(None, None, None, 0) == 3           # QM_ERR_INVALID_ARG
    null = None
    assert lib.qm_deltanet_decode(null, null, 1, 0, *([null] * 10), 0, null) == 3
    assert lib.qm_gqa_decode(null, null, 1, *([null] * 7), 1, null, 0, null, null, 1, null) == 3
    assert lib.qm_destroy(null) == 3


def test_no_device_is_a_clean_error():
    if M.device_count() > 0:
        pytest.skip("a device is visible")
    with pytest.raises(M.MixerError) as e:
        M.Context(0)
    assert e.value.code == 1


def test_rope_table_matches_oracle_bit_for_bit():
    O = load_oracle()
    c1, s1 = M.rope_table(8192 + 64)
    c2, s2 = O.rope_table(8192 + 64)
    assert np.array_equal(c1, c2) and np.array_equal(s1, s2)
    assert M.load_library().qm_rope_table(1e7, 63, 8, None, None) == 3


def test_workload_generators_are_seeded(workloads):
    a = workloads.dn_decode_workload(2, 1, seed=5)
    b = workloads.dn_decode_workload(2, 1, seed=5)
    assert all(np.array_equal(a[k], b[k]) for k in a)
    # decay g = exp(-softplus(a) * exp(A_log)) lies in (0, 1) with U(0.01, 0.1) rates
    rate = np.exp(a["a_log"].astype(np.float64))
    assert np.all((rate >= 0.01) & (rate <= 0.1))
    bits = workloads.bf16_bits(np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.0], np.float32))
    assert bits.tolist() == [0x3F80, 0x3F82, 0xC000]


def test_bench_refuses_more_than_one_gpu():
    """The bench measures one GPU; a request for more exits with a message
    before any device work."""
    import subprocess
    import sys
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=str(ROOT))
    assert r.returncode == 2
    assert "--gpus 1" in (r.stdout + r.stderr)
    assert not r.stdout.strip().startswith("{")
