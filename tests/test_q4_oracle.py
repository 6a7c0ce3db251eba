"""CPU pins of the oracle's Q4 functions (convert.rs:437-467 quantize_q4,
gemv.rs:412-445 gemv_q4_inner, :529-542 gemm_q4, :469-526 fused_gate_up_q4).

The reference has no tests or fixtures for these; the pins are a hand-worked
known answer (nibble order, code offset, scale = absmax / 7, rounding half
away from zero), the quantizer's error bound, exactness of one-hot products,
and float64 numpy products over an independent dequantization
(workloads.q4_dequant: numpy bit operations and numpy's f16).
"""
from __future__ import annotations

import numpy as np

from conftest import load_oracle, load_workloads

O = load_oracle()
W = load_workloads()


def test_quantize_known_answer():
    row = np.zeros((1, 64), np.float32)
    row[0, :4] = [-7.0, 7.0, 3.5, -3.5]   # absmax 7 -> scale 1; codes 1, 15, 12 (3.5 -> 4), 4 (-3.5 -> -4)
    row[0, 32 + 5] = 0.07                 # second group: scale 0.01, code 15 in the high nibble of byte 2
    packed, scales = O.q4_quantize(row)
    assert scales[0, 0] == 0x3C00         # f16 1.0
    assert scales[0, 1] == np.float16(np.float32(0.07) / np.float32(7.0)).view(np.uint16)
    assert list(packed[0, :3]) == [0xF1, 0x4C, 0x88]
    assert all(b == 0x88 for b in packed[0, 3:16])
    assert packed[0, 16 + 2] == 0xF8 and all(packed[0, 16 + j] == 0x88 for j in range(16) if j != 2)


def test_quantize_zero_group():
    packed, scales = O.q4_quantize(np.zeros((3, 32), np.float32))
    assert np.all(scales == 0) and np.all(packed == 0x88)


def test_quantize_error_bound():
    rng = np.random.default_rng(0)
    w = (0.02 * rng.standard_normal((64, 256))).astype(np.float32)
    packed, scales = O.q4_quantize(w)
    deq = W.q4_dequant(packed, scales).astype(np.float64)
    s32 = np.abs(w.reshape(64, 8, 32)).max(axis=2) / np.float32(7.0)
    s16 = W.f16_value(scales).astype(np.float64)
    bound = 0.5 * s32 + 8.0 * np.abs(s16 - s32) + 1e-12
    err = np.abs(deq - w).reshape(64, 8, 32).max(axis=2)
    assert np.all(err <= bound)
    # codes stay within -7..7 of the offset (absmax maps to +-7)
    q = np.concatenate([packed & 15, packed >> 4])
    assert q.min() >= 1 and q.max() <= 15


def test_gemv_one_hot_rows_exact():
    rng = np.random.default_rng(1)
    packed, scales = W.q4_random_weight(40, 96, rng)
    deq = W.q4_dequant(packed, scales)
    for k in (0, 17, 39):
        x = np.zeros(40, np.float32)
        x[k] = 1.0
        assert np.array_equal(O.q4_gemv(x, packed, scales), deq[k])


def test_gemv_matches_float64_product():
    rng = np.random.default_rng(2)
    for k, n in ((2560, 256), (300, 32), (1, 64)):
        packed, scales = W.q4_random_weight(k, n, rng)
        x = rng.standard_normal(k).astype(np.float32)
        x[::7] = 0.0                      # the reference skips zero inputs
        deq = W.q4_dequant(packed, scales).astype(np.float64)
        ref = x.astype(np.float64) @ deq
        mag = np.abs(x).astype(np.float64) @ np.abs(deq)
        got = O.q4_gemv(x, packed, scales)
        assert np.all(np.abs(got - ref) <= 1e-6 * mag + 1e-30)


def test_gemm_rows_and_gate_up():
    rng = np.random.default_rng(3)
    packed, scales = W.q4_random_weight(128, 64, rng)
    x = rng.standard_normal((5, 128)).astype(np.float32)
    y = O.q4_gemm(x, packed, scales)
    deq = W.q4_dequant(packed, scales).astype(np.float64)
    assert np.all(np.abs(y - x.astype(np.float64) @ deq) <= 1e-6 * (np.abs(x) @ np.abs(deq)) + 1e-30)
    up_p, up_s = W.q4_random_weight(128, 64, rng)
    out = O.q4_gate_up(x[0], packed, scales, up_p, up_s)
    g = x[0].astype(np.float64) @ deq
    u = x[0].astype(np.float64) @ W.q4_dequant(up_p, up_s).astype(np.float64)
    ref = g / (1.0 + np.exp(-g)) * u
    assert np.all(np.abs(out - ref) <= 1e-5 * np.abs(ref).max())


# ---- vocabulary side: lm_head_parallel (gemv.rs:678-708), embed_lookup_q4 (:544-563)
def _embed(vocab, hidden, seed):
    rng = np.random.default_rng(seed)
    packed, scales = W.q4_random_weight(vocab, hidden, rng, scale=0.02)
    return rng, packed, scales


def test_embed_known_answer_and_rows():
    """A hand-worked row (low nibble = even column, value s * (q - 8)), then
    every row equals the independent numpy dequantization bit for bit."""
    packed = np.full((2, 32), 0x88, np.uint8)
    scales = np.zeros((2, 2), np.uint16)
    packed[1, 0] = 0xF1                   # columns 0, 1: codes 1, 15 -> -7 s, 7 s
    packed[1, 17] = 0x0C                  # columns 34, 35: codes 12, 0 -> 4 s', -8 s'
    scales[1] = [0x3C00, 0x3800]          # s = 1, s' = 0.5
    row = O.q4_embed(packed, scales, 1)
    want = np.zeros(64, np.float32)
    want[:2] = [-7.0, 7.0]
    want[34:36] = [2.0, -4.0]
    assert np.array_equal(row, want)
    assert np.array_equal(O.q4_embed(packed, scales, 0), np.zeros(64, np.float32))
    _, packed, scales = _embed(300, 2560, 71)
    E = W.q4_dequant(packed, scales)
    for v in (0, 1, 157, 299):
        assert np.array_equal(O.q4_embed(packed, scales, v), E[v])


def test_lm_head_vs_float64_and_one_hot():
    """logits = E x within fp32 summation error of float64; a one-hot x
    reads one column of E exactly; a zero-scale group is skipped (an
    infinite x in it leaves that row finite, gemv.rs:685)."""
    rng, packed, scales = _embed(1000, 2560, 72)
    E = W.q4_dequant(packed, scales).astype(np.float64)
    x = rng.standard_normal(2560).astype(np.float32)
    got = O.q4_lm_head(x, packed, scales)
    ref = E @ x.astype(np.float64)
    mag = np.abs(E) @ np.abs(x).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 1e-5 * mag)
    oh = np.zeros(2560, np.float32)
    oh[1234] = 1.0
    assert np.array_equal(O.q4_lm_head(oh, packed, scales), E[:, 1234].astype(np.float32))
    scales = scales.copy()
    scales[5, 3] = 0
    xi = x.copy()
    xi[3 * 32 + 7] = np.inf
    out = O.q4_lm_head(xi, packed, scales)
    assert np.isfinite(out[5]) and not np.isfinite(out[6])
