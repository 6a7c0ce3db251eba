"""CPU pins of the oracle's sampling (generate.rs:41-82,334-384 and the wgpu
twin gpu_inference.rs:855-931).

The reference has no tests for these.  Pins: the published first output of
Marsaglia's xorshift64 (13, 7, 17) from his example seed, the generator as
a GF(2)-linear map built from shift matrices, hand-worked penalty cases,
numpy's stable argsort and float64 softmax for the top-k and its
probabilities, the cumulative-draw bracket, and empirical frequencies.
"""
from __future__ import annotations

import numpy as np

from conftest import load_oracle

O = load_oracle()
M64 = (1 << 64) - 1


def test_xorshift64_known_answer_and_linear_form():
    st = np.array([88172645463325252], np.uint64)          # Marsaglia (2003), xor64 example seed
    r = O.rng_next_f32(st)
    assert int(st[0]) == 8748534153485358512
    assert r == np.float32((8748534153485358512 >> 40) / 2.0 ** 24)

    def shift_matrix(n, left):
        m = np.zeros((64, 64), np.uint8)
        for i in range(64):
            j = i + n if left else i - n                    # bit i of the input moves to bit j
            if 0 <= j < 64:
                m[j, i] = 1
        return m

    eye = np.eye(64, dtype=np.uint8)
    T = eye
    for n, left in ((13, True), (7, False), (17, True)):
        T = ((eye + shift_matrix(n, left)) % 2) @ T % 2
    rng = np.random.default_rng(1)
    for _ in range(20):
        s0 = int(rng.integers(1, 1 << 63)) * 2 + 1
        bits = np.array([(s0 >> i) & 1 for i in range(64)], np.uint8)
        want = sum(int(b) << i for i, b in enumerate(T @ bits % 2))
        st = np.array([s0], np.uint64)
        O.rng_next_f32(st)
        assert int(st[0]) == want


def test_penalties_known_answers():
    logits = np.array([2.0, -2.0, 0.5, 3.0, 1.0], np.float32)
    gen = [3] * 3 + [9, -1] + [4] * 59 + [0, 1, 0]          # 67 ids: the 3s fall outside the 64-id window
    out = O.apply_penalties(logits, gen, 2.0, 0.0)
    assert list(out) == [0.5, -4.0, 0.5, 3.0, 1.0 / 2.0 ** 59]
    out = O.apply_penalties(logits, gen, 1.0, 1.5)           # presence only, once per distinct id
    assert list(out) == [0.5, -3.5, 0.5, 1.5, -0.5]
    out = O.apply_penalties(logits, [], 2.0, 1.5)
    assert np.array_equal(out, logits)


def test_greedy_first_and_last_maximum():
    x = np.array([1.0, 5.0, -2.0, 5.0, 0.0], np.float32)
    st = np.array([7], np.uint64)
    assert O.sample_top_k(x, 0.0, 0.9, 20, st)[0] == 1 == int(np.argmax(x))
    assert O.sample_top_k(x, 0.0, 0.9, 20, st, wgpu=True)[0] == 3
    assert int(st[0]) == 7                                   # no draw


def test_top_k_ids_probs_and_draw_bracket():
    rng = np.random.default_rng(3)
    x = np.round(2.0 * rng.standard_normal(5000), 1).astype(np.float32)   # many ties
    for temp, top_p, top_k in ((1.0, 0.95, 20), (0.7, 0.5, 50), (1.3, 1.0, 300)):
        st = np.array([12345678901234567], np.uint64)
        s0 = int(st[0])
        tok, ids, probs = O.sample_top_k(x, temp, top_p, top_k, st)
        order = np.argsort(-x, kind="stable")[:top_k]
        assert np.array_equal(ids, order)
        z = (x[order].astype(np.float64) - x.max()) / temp
        p64 = np.exp(z) / np.exp(z).sum()
        assert np.allclose(probs, p64, rtol=2e-6, atol=0)
        c = np.cumsum(p64)
        cutoff = int(np.searchsorted(c, top_p - 1e-6)) + 1
        s = s0                                               # one xorshift64 step
        s ^= (s << 13) & M64
        s ^= s >> 7
        s ^= (s << 17) & M64
        assert int(st[0]) == s
        u = (s >> 40) / 2.0 ** 24 * c[cutoff - 1]
        j = int(np.searchsorted(c[:cutoff], u))
        assert tok == order[min(j, cutoff - 1)]


def test_empirical_frequencies():
    x = np.array([3.0, 2.5, 2.0, 1.0, -1.0, 0.0], np.float32)
    st = np.array([99991], np.uint64)
    n = 20000
    counts = np.zeros(x.size)
    for _ in range(n):
        counts[O.sample_top_k(x, 1.0, 1.0, 4, st)[0]] += 1
    _, ids, probs = O.sample_top_k(x, 1.0, 1.0, 4, st)
    assert counts[4] == counts[5] == 0
    for i, p in zip(ids, probs):
        assert abs(counts[i] / n - p) < 4.0 * np.sqrt(p * (1 - p) / n)
