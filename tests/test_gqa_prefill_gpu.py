"""GPU parity: GQA causal prefill (qm_gqa_prefill) vs the CPU oracle.

The oracle restates gemv.rs:1364-1444 in fp32 on the same bf16-rounded
inputs.  Bar (bf16 path): ||d||_inf / ||ref||_inf <= 2e-2 on the gated
output rows; the f16 K cache within one f16 step of the oracle's normed and
rotated K, the f16 V cache exactly the f16 rounding of v.  At seq 8192 the oracle runs on
a row subset (first, last and spread rows) to stay within seconds.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import load_mixer, load_oracle, load_workloads

pytestmark = pytest.mark.gpu

M = load_mixer()
O = load_oracle()
W = load_workloads()
RTOL = 2e-2


def run_gpu(ctx, w, S, cap):
    cos, sin = M.rope_table(max(S, 1))
    d = {k: ctx.upload(w[k]) for k in ["q_gate", "k", "v", "q_norm", "k_norm"]}
    rc, rs = ctx.upload(cos), ctx.upload(sin)
    kc = ctx.alloc(4 * cap * 256 * 2)
    vc = ctx.alloc(4 * cap * 256 * 2)
    out = ctx.alloc(S * 16 * 256 * 2)
    ctx.gqa_prefill(S, d["q_gate"], d["k"], d["v"], d["q_norm"], d["k_norm"], rc, rs, S, kc, vc, cap, out)
    o = W.bf16_value(ctx.download(out, (S, 16, 256), np.uint16))
    K = ctx.download(kc, (4, cap, 256), np.uint16)[:, :S]
    V = ctx.download(vc, (4, cap, 256), np.uint16)[:, :S]
    return o, K, V


def run_oracle(w, S, rows=None):
    cfg = O.config()
    cos, sin = O.rope_table(S)
    out, kc, vc = O.attn_prefill(cfg, W.bf16_value(w["q_gate"]).reshape(S, -1),
                                 W.bf16_value(w["k"]).reshape(S, -1), W.bf16_value(w["v"]).reshape(S, -1),
                                 w["q_norm"], w["k_norm"], cos, sin, rows=rows, nthreads=8)
    return out.reshape(S, 16, 256), kc, vc


def check(o, K, V, ref, kc, vc, rows):
    err = float(np.abs(o[rows] - ref[rows]).max() / np.abs(ref[rows]).max())
    kgot = W.f16_value(K).transpose(1, 0, 2)
    kerr = np.abs(kgot - kc)
    print(f"rel out {err:.3e}  max|dK| {kerr.max():.3e}")
    assert err <= RTOL
    assert np.all(kerr <= np.abs(kc) * 2 ** -10 + 1e-6)
    # V is stored as the f16 rounding of the bf16 input (not exact below f16's normal range)
    assert np.array_equal(W.f16_value(V).transpose(1, 0, 2), W.f16_value(W.f16_bits(vc)))


@pytest.mark.parametrize("S", [1, 37, 64, 200])
def test_prefill_small(ctx, S):
    w = W.gqa_prefill_workload(S, seed=3 + S)
    print(f"case: gqa prefill S={S}", flush=True)
    o, K, V = run_gpu(ctx, w, S, S + 5)
    ref, kc, vc = run_oracle(w, S)
    check(o, K, V, ref, kc, vc, np.arange(S))


def test_prefill_8192_rows(ctx):
    """Rows checked: the first 40 and last 24, 40 evenly spaced, 256 drawn
    at random over the whole triangle, and the rows on both sides of the
    48-row block and 64-key tile edges around the middle (the K and V caches
    are checked in full)."""
    S = 8192
    w = W.gqa_prefill_workload(S, seed=3)
    print("case: gqa prefill S=8192", flush=True)
    o, K, V = run_gpu(ctx, w, S, S)
    mid = [e + d for e in (4080, 4128, 4096, 4160) for d in (-1, 0, 1)]
    rows = np.unique(np.concatenate([np.arange(0, 40), np.arange(S - 24, S),
                                     np.linspace(0, S - 1, 40).astype(np.int64),
                                     np.random.default_rng(5).integers(0, S, 256), mid]))
    ref, kc, vc = run_oracle(w, S, rows=rows)
    check(o, K, V, ref, kc, vc, rows)


def test_prefill_5000_rows(ctx):
    """S = 5000, a multiple of neither the 48-row block nor the 64-key tile:
    the last tile copy is zero padded past S, and the last row block is
    partial.  Checked on the last 60 rows, 120 random rows and the first 20."""
    S = 5000
    w = W.gqa_prefill_workload(S, seed=23)
    print("case: gqa prefill S=5000", flush=True)
    o, K, V = run_gpu(ctx, w, S, S + 3)
    rows = np.unique(np.concatenate([np.arange(0, 20), np.arange(S - 60, S),
                                     np.random.default_rng(7).integers(0, S, 120)]))
    ref, kc, vc = run_oracle(w, S, rows=rows)
    check(o, K, V, ref, kc, vc, rows)


@pytest.mark.parametrize("S", [8192, 10000, 5000])
def test_prefill_block_order(ctx, S):
    """The packed row-block order (QM_OPT_GQA_PREFILL_ORDER = 2; at 8192 and
    10000 tokens also the automatic one) and longest first give bit-identical
    outputs on every row: each block is computed once, by whichever
    workgroup draws it.  The output starts as NaN, so a block left out
    would show."""
    w = W.gqa_prefill_workload(S, seed=41)
    print(f"case: gqa prefill block order S={S}", flush=True)
    cos, sin = M.rope_table(S)
    d = {k: ctx.upload(w[k]) for k in ["q_gate", "k", "v", "q_norm", "k_norm"]}
    rc, rs = ctx.upload(cos), ctx.upload(sin)
    outs = []
    try:
        for mode in (1, 2, 0):
            ctx.set_option(M.QM_OPT_GQA_PREFILL_ORDER, mode)
            kc = ctx.alloc(4 * S * 256 * 2)
            vc = ctx.alloc(4 * S * 256 * 2)
            out = ctx.upload(np.full((S, 16, 256), 0x7FC0, np.uint16))
            ctx.gqa_prefill(S, d["q_gate"], d["k"], d["v"], d["q_norm"], d["k_norm"], rc, rs, S, kc, vc, S, out)
            outs.append(ctx.download(out, (S, 16, 256), np.uint16))
    finally:
        ctx.set_option(M.QM_OPT_GQA_PREFILL_ORDER, 0)
    assert not np.isnan(W.bf16_value(outs[0])).any()
    assert np.array_equal(outs[0], outs[1])
    assert np.array_equal(outs[0], outs[2])


def test_prefill_score_jumps(ctx):
    """Later keys that score far above the earlier ones: every query is one
    vector b; keys from position 150 lean 60% towards b (a jump of well over
    8 in log2 units, so the running max moves and O is rescaled) and keys
    from 700 are b itself (a smaller second jump that stays under the
    reference max's slack, so P grows to ~2^7 before normalisation)."""
    S = 1000
    w = W.gqa_prefill_workload(S, seed=11)
    rng = np.random.default_rng(12)
    b = rng.standard_normal(256).astype(np.float32)
    qg = W.bf16_value(w["q_gate"]).reshape(S, 16, 512).copy()
    qg[:, :, :256] = b
    k = W.bf16_value(w["k"]).reshape(S, 4, 256).copy()
    k[150:700] = 0.6 * b + 0.4 * k[150:700]
    k[700:] = b
    w["q_gate"] = W.bf16_bits(qg.reshape(w["q_gate"].shape))
    w["k"] = W.bf16_bits(k.reshape(w["k"].shape))
    print("case: gqa prefill S=1000 score jumps", flush=True)
    o, K, V = run_gpu(ctx, w, S, S)
    ref, kc, vc = run_oracle(w, S)
    check(o, K, V, ref, kc, vc, np.arange(S))


@pytest.mark.parametrize("scale", [1e3, 3e4])
def test_prefill_value_outliers(ctx, scale):
    """v channels times `scale` / 4 (|v| up to ~3e4 at 3e4, inside f16's
    range, which the configured f16 KV cache sets for the whole GQA path)
    and q/k channels likewise (RMS-normalised per head, so they only sharpen
    the scores)."""
    S = 300
    w = W.gqa_prefill_workload(S, seed=17)
    v = W.bf16_value(w["v"]).reshape(S, 4, 256).copy()
    v[:, :, [3, 100, 255]] *= np.float32(scale / 4)      # |v| up to ~3e4, below f16's 65504
    k = W.bf16_value(w["k"]).reshape(S, 4, 256).copy()
    k[:, :, [9, 200]] *= np.float32(scale)
    w["v"] = W.bf16_bits(v.reshape(w["v"].shape))
    w["k"] = W.bf16_bits(k.reshape(w["k"].shape))
    print(f"case: gqa prefill S={S} value outliers x{scale:g}", flush=True)
    o, K, V = run_gpu(ctx, w, S, S)
    ref, kc, vc = run_oracle(w, S)
    assert np.isfinite(o).all()
    check(o, K, V, ref, kc, vc, np.arange(S))


@pytest.mark.parametrize("S,order", [(2000, 0), (8192, 2)])
def test_prefill_graph_replay_matches_eager(ctx, S, order):
    """A captured prefill (K/V kernel, which resets the row-block queues, then
    the persistent attention) replayed several times, with eager prefills and
    synchronisations in between, matches the eager output bit for bit: which
    workgroup takes which row block does not change the arithmetic.  At 8192
    tokens the packed order travels in the captured kernel arguments, and
    the eager prefills in between run another length (another plan), which
    must not disturb the captured one."""
    w = W.gqa_prefill_workload(S, seed=17)
    cos, sin = M.rope_table(S)
    d = {k: ctx.upload(w[k]) for k in ["q_gate", "k", "v", "q_norm", "k_norm"]}
    rc, rs = ctx.upload(cos), ctx.upload(sin)
    kc, vc = ctx.alloc(4 * S * 256 * 2), ctx.alloc(4 * S * 256 * 2)
    out_e, out_g = ctx.alloc(S * 16 * 256 * 2), ctx.alloc(S * 16 * 256 * 2)
    ctx.reserve(max_batch=1, max_prefill_tokens=S)
    other = S - 1000                      # the eager length run between replays

    def run(out, n=S):
        ctx.gqa_prefill(n, d["q_gate"], d["k"], d["v"], d["q_norm"], d["k_norm"], rc, rs, S, kc, vc, S, out)

    ctx.set_option(M.QM_OPT_GQA_PREFILL_ORDER, order)
    try:
        print(f"case: gqa prefill graph replay S={S} order={order} (eager reference)", flush=True)
        run(out_e)
        ref = ctx.download(out_e, (S, 16 * 256), np.uint16)
        ctx.graph_begin()
        run(out_g)
        g = ctx.graph_end()
        for rep in range(3):
            print(f"case: gqa prefill graph replay S={S} order={order} rep {rep}", flush=True)
            ctx.fill_normal(out_g, M.QM_BF16, S * 16 * 256, 0.0, 1.0, seed=rep)   # poison between replays
            g.launch()
            ctx.sync()
            assert np.array_equal(ctx.download(out_g, (S, 16 * 256), np.uint16), ref)
            run(out_e, other)                                                # eager work in between
            ctx.sync()
        g.close()
    finally:
        ctx.set_option(M.QM_OPT_GQA_PREFILL_ORDER, 0)
