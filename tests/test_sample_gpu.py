"""GPU parity: next-token sampling (qm_sample) vs the oracle's restatement of
generate.rs:58-82,334-384 and of the wgpu twin (gpu_inference.rs:867-931).

Integer results are compared exactly: the token, the xorshift64 state after
the step and the sorted top-k ids.  Penalized logits are bit-identical.
Probabilities: within 2 ulp of the oracle's (exp is correctly rounded on
the device; libm's expf can differ by an ulp).  Logits come at the full
248,320-entry vocabulary, some rounded to 0.25 steps so that ties (and
-0 / +0) are common and the index order of equal logits is exercised.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import load_mixer, load_oracle

pytestmark = pytest.mark.gpu

M = load_mixer()
O = load_oracle()
VOCAB = 248320


def _logits(rng, tied):
    x = 3.0 * rng.standard_normal(VOCAB)
    if tied:
        x = np.round(4.0 * x) / 4.0
        x[rng.integers(0, VOCAB, 50)] = -0.0
    return x.astype(np.float32)


def _run(ctx, x, state0, steps, temp, top_p, top_k, wgpu):
    """steps draws from the same logits with the state carried on the device."""
    k = 1 if temp <= 0 else min(top_k, VOCAB)
    dx, dst = ctx.upload(x), ctx.upload(np.array([state0], np.uint64))
    tok, ids, probs = ctx.alloc(4), ctx.alloc(4 * k), ctx.alloc(4 * k)
    st = np.array([state0], np.uint64)
    flags = M.QM_SAMPLE_WGPU if wgpu else 0
    for s in range(steps):
        ctx.sample(VOCAB, dx, None, 0, dst, tok, temperature=temp, top_p=top_p, top_k=top_k, flags=flags,
                   top_ids=ids, top_probs=probs)
        want, wids, wprobs = O.sample_top_k(x, temp, top_p, top_k, st, wgpu=wgpu)
        got = int(ctx.download(tok, (1,), np.int32)[0])
        gst = int(ctx.download(dst, (1,), np.uint64)[0])
        assert (got, gst) == (want, int(st[0])), f"step {s}"
        assert np.array_equal(ctx.download(ids, (k,), np.int32), wids[:k])
        if temp > 0:
            gp = ctx.download(probs, (k,), np.float32)
            assert np.all(np.abs(gp - wprobs) <= 2 * np.spacing(wprobs))


@pytest.mark.parametrize("temp,top_p,top_k,tied,wgpu", [
    (1.0, 0.95, 20, False, False), (0.7, 0.9, 50, True, False), (1.3, 1.0, 1024, True, False),
    (1.0, 0.5, 1, False, False), (1.0, 0.95, 20, True, True), (0.0, 0.95, 20, True, False),
    (0.0, 0.95, 20, True, True), (2.0, 0.999, 300, False, True)])
def test_sample_matches_oracle(ctx, temp, top_p, top_k, tied, wgpu):
    rng = np.random.default_rng(int(1000 * temp) + top_k + 7 * tied + 13 * wgpu)
    x = _logits(rng, tied)
    print(f"case: sample T={temp} p={top_p} k={top_k} tied={tied} wgpu={wgpu}", flush=True)
    _run(ctx, x, 0x9E3779B97F4A7C15, 25 if temp > 0 else 2, temp, top_p, top_k, wgpu)


def test_sample_all_equal_and_small_vocab(ctx):
    """Every logit equal: the first top_k indices in order, uniform
    probabilities; a vocabulary smaller than top_k."""
    x = np.full(VOCAB, 1.5, np.float32)
    _run(ctx, x, 5, 3, 1.0, 0.95, 64, False)
    small = np.array([0.5, -1.0, 2.0], np.float32)
    dx, dst = ctx.upload(small), ctx.upload(np.array([77], np.uint64))
    tok = ctx.alloc(4)
    st = np.array([77], np.uint64)
    for _ in range(10):
        ctx.sample(3, dx, None, 0, dst, tok, temperature=1.0, top_p=1.0, top_k=20)
        assert int(ctx.download(tok, (1,), np.int32)[0]) == O.sample_top_k(small, 1.0, 1.0, 20, st)[0]
    assert int(ctx.download(dst, (1,), np.uint64)[0]) == int(st[0])


def test_penalties_in_place(ctx):
    """generate.rs:58-82 then the think-block EOS ban (generate.rs:191)."""
    rng = np.random.default_rng(5)
    x = _logits(rng, False)
    gen = rng.integers(0, VOCAB, 300).astype(np.int32)
    gen[-64:-40] = gen[-10]                               # repeats inside the window
    gen[5] = VOCAB + 3                                    # out of range: ignored
    gen[6] = -4
    dx, dg = ctx.upload(x), ctx.upload(gen)
    dst, tok = ctx.upload(np.array([3], np.uint64)), ctx.alloc(4)
    print("case: penalties", flush=True)
    ctx.sample(VOCAB, dx, dg, len(gen), dst, tok, temperature=0.8, top_p=0.95, top_k=20,
               repetition_penalty=1.3, presence_penalty=1.5, banned_id=int(np.argmax(x)))
    want = O.apply_penalties(x, gen, 1.3, 1.5)
    want[int(np.argmax(x))] = -np.inf
    assert np.array_equal(ctx.download(dx, (VOCAB,), np.float32), want)
    st = np.array([3], np.uint64)
    assert int(ctx.download(tok, (1,), np.int32)[0]) == O.sample_top_k(want, 0.8, 0.95, 20, st)[0]


def test_sample_errors(ctx):
    dx, dst, tok = ctx.alloc(64), ctx.upload(np.array([1], np.uint64)), ctx.alloc(4)
    for kw in ({"top_k": 0}, {"top_k": 1025}, {"flags": 6}):
        with pytest.raises(M.MixerError) as e:
            ctx.sample(16, dx, None, 0, dst, tok, temperature=1.0, **kw)
        assert e.value.code == 3
    with pytest.raises(M.MixerError) as e:             # beyond the presence bitmap
        ctx.sample(262145, dx, None, 0, dst, tok, temperature=1.0)
    assert e.value.code == 4
    with pytest.raises(M.MixerError) as e:             # wgpu twin: top_k above the vocabulary
        ctx.sample(16, dx, None, 0, dst, tok, temperature=1.0, top_k=20, flags=M.QM_SAMPLE_WGPU)
    assert e.value.code == 3


def test_sample_in_graph_replays(ctx):
    """The penalties, top-k select and draw captured once as a HIP graph and
    replayed five times, with eager work on the same logits buffer between
    replays (a fresh upload each time): every replay's token and xorshift64
    state equal the oracle's sequence, as eager calls do."""
    rng = np.random.default_rng(91)
    ctx.reserve(1, 0, 0)
    dx = ctx.alloc(VOCAB * 4)
    gen = rng.integers(0, VOCAB, 200).astype(np.int32)
    dg, dst, tok = ctx.upload(gen), ctx.upload(np.array([2024], np.uint64)), ctx.alloc(16)
    st = np.array([2024], np.uint64)
    kw = dict(temperature=0.9, top_p=0.9, top_k=40, repetition_penalty=1.2, presence_penalty=1.0)
    ctx.sync()
    ctx.graph_begin()
    ctx.sample(VOCAB, dx, dg, len(gen), dst, tok, **kw)
    g = ctx.graph_end()
    print("case: sample graph replays", flush=True)
    for rep in range(5):
        x = _logits(rng, rep % 2 == 1)
        ctx.upload(x, dx)                                  # eager work between replays
        g.launch()
        ctx.sync()
        want = O.sample_top_k(O.apply_penalties(x, gen, 1.2, 1.0), 0.9, 0.9, 40, st)[0]
        got = int(ctx.download(tok, (1,), np.int32)[0])
        assert (got, int(ctx.download(dst, (1,), np.uint64)[0])) == (want, int(st[0])), f"replay {rep}"
    g.close()
