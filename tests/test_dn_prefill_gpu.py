"""GPU parity: DeltaNet chunked prefill (qm_deltanet_prefill).

Checked against (a) the oracle's sequential prefill (gemv.rs:1119-1219) on
the same bf16-rounded inputs and (b) seq_len recurrent steps of the GPU
decode kernel in layer mode (conv1d + SiLU in-kernel), the chunked form's
own criterion.  Bar (bf16 path): ||d||_inf / ||ref||_inf <= 2e-2 for the
outputs and the final state; the conv buffer is exact.
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


def rel(got, ref):
    return float(np.abs(got.astype(np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


def run_prefill(ctx, w, T):
    up = ctx.upload
    d = {k: up(w[k]) for k in ["qkv", "conv_w", "a", "b", "a_log", "dt_bias", "z", "norm_w"]}
    state = up(w["state0"])
    buf = up(w["conv_buf0"])
    out = ctx.alloc(T * 4096 * 2)
    ctx.deltanet_prefill(T, d["qkv"], buf, d["conv_w"], d["a"], d["b"], d["a_log"], d["dt_bias"],
                         d["z"], d["norm_w"], state, out)
    o = W.bf16_value(ctx.download(out, (T, 4096), np.uint16))
    S = ctx.download(state, (32, 128, 128), np.float32)
    cb = ctx.download(buf, (8192, 3), np.float32)
    return o, S, cb


def run_oracle(w, T):
    cfg = O.config()
    S = w["state0"].copy()
    buf = w["conv_buf0"].copy()
    out = O.deltanet_prefill(cfg, W.bf16_value(w["qkv"]), w["a"], w["b"], W.bf16_value(w["z"]),
                             w["conv_w"], w["a_log"], w["dt_bias"], w["norm_w"], S, buf)
    return out, S, buf


@pytest.mark.parametrize("T,warm", [(256, False), (100, True), (1, True), (65, True)])
def test_prefill_vs_oracle(ctx, T, warm):
    w = W.dn_prefill_workload(T, seed=2 + T)
    if warm:   # nonzero entering state and conv history
        r = np.random.default_rng(T)
        w["state0"] = (0.02 * r.standard_normal((32, 128, 128))).astype(np.float32)
        w["conv_buf0"] = r.standard_normal((8192, 3)).astype(np.float32)
    print(f"case: dn prefill T={T} warm={warm}", flush=True)
    o, S, cb = run_prefill(ctx, w, T)
    ro, rS, rcb = run_oracle(w, T)
    eo, es = rel(o, ro), rel(S, rS)
    print(f"rel out {eo:.3e} rel state {es:.3e}")
    assert eo <= RTOL and es <= RTOL
    assert np.array_equal(cb, rcb)


def test_prefill_4096_vs_oracle_and_recurrent_decode(ctx):
    """seq 4096, zero initial state: chunked == 4096 recurrent steps."""
    T = 4096
    w = W.dn_prefill_workload(T, seed=2)
    print("case: dn prefill T=4096 vs oracle", flush=True)
    o, S, cb = run_prefill(ctx, w, T)
    ro, rS, rcb = run_oracle(w, T)
    eo, es = rel(o, ro), rel(S, rS)
    print(f"vs oracle: rel out {eo:.3e} rel state {es:.3e}")
    assert eo <= RTOL and es <= RTOL
    assert np.array_equal(cb, rcb)

    # the decode kernel, one launch per token, layer mode
    print("case: dn decode x4096 (layer mode)", flush=True)
    up = ctx.upload
    qkv = up(W.bf16_value(w["qkv"]))
    z = up(W.bf16_value(w["z"]))
    a, b = up(w["a"]), up(w["b"])
    conv_w, a_log, dt_bias, norm_w = up(w["conv_w"]), up(w["a_log"]), up(w["dt_bias"]), up(w["norm_w"])
    state = up(w["state0"])
    buf = up(w["conv_buf0"])
    out = ctx.alloc(T * 4096 * 4)
    for t in range(T):
        ctx.deltanet_decode(1, M.QM_DN_PREACT, qkv.offset(t * 8192 * 4), buf, conv_w, a.offset(t * 32 * 4),
                            b.offset(t * 32 * 4), a_log, dt_bias, z.offset(t * 4096 * 4), norm_w, state,
                            out.offset(t * 4096 * 4))
    od = ctx.download(out, (T, 4096), np.float32)
    Sd = ctx.download(state, (32, 128, 128), np.float32)
    e1, e2 = rel(o, od), rel(S, Sd)
    print(f"vs recurrent decode: rel out {e1:.3e} rel state {e2:.3e}")
    assert e1 <= RTOL and e2 <= RTOL
    assert np.array_equal(ctx.download(buf, (8192, 3), np.float32), cb)


@pytest.mark.parametrize("T", [1500, 2500, 8292])
def test_prefill_long_warm(ctx, T):
    """Longer sequences from a nonzero entering state and conv history: 24,
    40 and 130 chunks (8292: more than one 64-chunk window of the scan's
    gamma loads, and a partial last chunk)."""
    w = W.dn_prefill_workload(T, seed=7 + T)
    r = np.random.default_rng(T)
    w["state0"] = (0.02 * r.standard_normal((32, 128, 128))).astype(np.float32)
    w["conv_buf0"] = r.standard_normal((8192, 3)).astype(np.float32)
    print(f"case: dn prefill warm T={T}", flush=True)
    o, S, cb = run_prefill(ctx, w, T)
    ro, rS, rcb = run_oracle(w, T)
    eo, es = rel(o, ro), rel(S, rS)
    print(f"rel out {eo:.3e} rel state {es:.3e}")
    assert eo <= RTOL and es <= RTOL
    assert np.array_equal(cb, rcb)


@pytest.mark.parametrize("scale", [1e3, 1e4])
def test_prefill_channel_outliers(ctx, scale):
    """A few input channels scaled far past the rest (massive-activation
    outliers): 4 v channels and 4 q/k channels times `scale` over 1024
    tokens.  q and k are L2-normalised per head, so their outliers only
    sharpen the direction; v's reach the f16 chunk operands and the state
    (|S| to ~6e3 at 1e4).  Within the bar against the oracle's fp32."""
    T = 1024
    w = W.dn_prefill_workload(T, seed=11)
    x = W.bf16_value(w["qkv"]).copy()
    x[:, [4096 + 5, 4096 + 900, 4096 + 2100, 4096 + 4000]] *= np.float32(scale)
    x[:, [7, 300, 2048 + 11, 2048 + 1500]] *= np.float32(scale)
    w["qkv"] = W.bf16_bits(x)
    print(f"case: dn prefill T={T} channel outliers x{scale:g}", flush=True)
    o, S, cb = run_prefill(ctx, w, T)
    ro, rS, rcb = run_oracle(w, T)
    assert np.isfinite(o).all() and np.isfinite(S).all()
    eo, es = rel(o, ro), rel(S, rS)
    print(f"rel out {eo:.3e} rel state {es:.3e} max|S| {np.abs(rS).max():.3e}")
    assert eo <= RTOL and es <= RTOL
    assert np.array_equal(cb, rcb)


def test_prefill_slow_decay(ctx):
    """Decays near 1 (A_log = log 1e-4: alpha ~ 0.9999 per token) over 1024
    tokens, so the chunk-local cumulative decays stay ~1 and the state keeps
    every token's contribution."""
    T = 1024
    w = W.dn_prefill_workload(T, seed=13)
    w["a_log"] = np.full(32, np.log(1e-4), np.float32)
    print(f"case: dn prefill T={T} slow decay", flush=True)
    o, S, cb = run_prefill(ctx, w, T)
    ro, rS, rcb = run_oracle(w, T)
    eo, es = rel(o, ro), rel(S, rS)
    print(f"rel out {eo:.3e} rel state {es:.3e}")
    assert eo <= RTOL and es <= RTOL


def test_prefill_graph_replay_matches_eager(ctx):
    """The prefill captured in a graph replays to the eager result, bit for
    bit, three times (state and conv buffer reset between replays)."""
    T = 2500
    w = W.dn_prefill_workload(T, seed=31)
    up = ctx.upload
    d = {k: up(w[k]) for k in ["qkv", "conv_w", "a", "b", "a_log", "dt_bias", "z", "norm_w"]}
    state, buf = up(w["state0"]), up(w["conv_buf0"])
    out = ctx.alloc(T * 4096 * 2)

    def call():
        ctx.deltanet_prefill(T, d["qkv"], buf, d["conv_w"], d["a"], d["b"], d["a_log"], d["dt_bias"],
                             d["z"], d["norm_w"], state, out)

    print("case: dn prefill graph replay T=2500", flush=True)
    ctx.reserve(max_batch=1, max_prefill_tokens=T)
    call()
    ctx.sync()
    ref_o = ctx.download(out, (T, 4096), np.uint16)
    ref_S = ctx.download(state, (32, 128, 128), np.float32)
    ctx.graph_begin()
    call()
    g = ctx.graph_end()
    for rep in range(3):
        up(w["state0"], state)
        up(w["conv_buf0"], buf)
        ctx.memset(out, 0, T * 4096 * 2)
        ctx.sync()
        g.launch()
        ctx.sync()
        assert np.array_equal(ctx.download(out, (T, 4096), np.uint16), ref_o), rep
        assert np.array_equal(ctx.download(state, (32, 128, 128), np.float32), ref_S), rep
