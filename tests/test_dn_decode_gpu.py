"""GPU parity: DeltaNet decode step (qm_deltanet_decode) vs the CPU oracle.

The oracle is the C restatement of gemv.rs:744-883 (AVX-512 head update when
the host has it, as the reference dispatches at gemv.rs:814-834).  Bar:
max-abs <= 1e-3 on the fp32 outputs and state.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import load_mixer, load_oracle, load_workloads

pytestmark = pytest.mark.gpu

M = load_mixer()
O = load_oracle()
W = load_workloads()
TOL = 1e-3
HEAD = 32 * 128 * 128


class DnDevice:
    """Device copies of a DeltaNet decode workload."""

    def __init__(self, ctx, w, steps, batch):
        self.ctx, self.steps, self.batch = ctx, steps, batch
        up = ctx.upload
        self.qkv = up(w["qkv"][:steps])
        self.a = up(w["a"][:steps])
        self.b = up(w["b"][:steps])
        self.z = up(w["z"][:steps])
        self.a_log, self.dt_bias = up(w["a_log"]), up(w["dt_bias"])
        self.norm_w, self.conv_w = up(w["norm_w"]), up(w["conv_w"])
        self.state = up(w["state0"])
        self.conv_buf = up(w["conv_buf0"])
        self.out = ctx.alloc(steps * batch * 4096 * 4)

    def step(self, t, flags=M.QM_DN_POSTACT):
        B = self.batch
        self.ctx.deltanet_decode(
            B, flags, self.qkv.offset(t * B * 8192 * 4), self.conv_buf, self.conv_w,
            self.a.offset(t * B * 32 * 4), self.b.offset(t * B * 32 * 4), self.a_log, self.dt_bias,
            self.z.offset(t * B * 4096 * 4), self.norm_w, self.state, self.out.offset(t * B * 4096 * 4))

    def outputs(self):
        return self.ctx.download(self.out, (self.steps, self.batch, 4096), np.float32)

    def final_state(self):
        return self.ctx.download(self.state, (self.batch, 32, 128, 128), np.float32)


def oracle_run(w, steps, batch, preact=False):
    cfg = O.config()
    outs = np.empty((steps, batch, 4096), np.float32)
    states = []
    for bi in range(batch):
        S = w["state0"][bi].copy()
        buf = w["conv_buf0"][bi].copy()
        for t in range(steps):
            outs[t, bi] = O.deltanet_decode_step(cfg, w["qkv"][t, bi], w["a"][t, bi], w["b"][t, bi],
                                                 w["z"][t, bi], w["conv_w"], w["a_log"], w["dt_bias"],
                                                 w["norm_w"], S, buf, preact=preact)
        states.append(S)
    return outs, np.stack(states)


def test_decode_256_steps_batch1(ctx):
    """256 sequential steps at batch 1, activated inputs, vs the oracle."""
    steps = 256
    w = W.dn_decode_workload(steps, 1, seed=0)
    print("case: dn decode B=1 steps=256 seed=0", flush=True)
    dev = DnDevice(ctx, w, steps, 1)
    for t in range(steps):
        dev.step(t)
    got, S = dev.outputs(), dev.final_state()
    ref, Sref = oracle_run(w, steps, 1)
    err_o = np.abs(got - ref).max()
    err_s = np.abs(S - Sref).max()
    print(f"max|dout|={err_o:.3e} max|dS|={err_s:.3e}")
    assert err_o <= TOL and err_s <= TOL


def test_decode_layer_mode_conv(ctx):
    """Layer mode: raw projections through conv1d+SiLU with the conv buffer."""
    steps = 12
    w = W.dn_decode_workload(steps, 2, seed=3)
    w["conv_buf0"] = (0.5 * np.random.default_rng(4).standard_normal(w["conv_buf0"].shape)).astype(np.float32)
    print("case: dn decode layer mode B=2 steps=12", flush=True)
    dev = DnDevice(ctx, w, steps, 2)
    for t in range(steps):
        dev.step(t, M.QM_DN_PREACT)
    got, S = dev.outputs(), dev.final_state()
    buf = ctx.download(dev.conv_buf, w["conv_buf0"].shape, np.float32)
    ref, Sref = oracle_run(w, steps, 2, preact=True)
    print(f"max|dout|={np.abs(got - ref).max():.3e} max|dS|={np.abs(S - Sref).max():.3e}")
    assert np.abs(got - ref).max() <= TOL and np.abs(S - Sref).max() <= TOL
    # the buffer holds the last three raw inputs exactly
    assert np.array_equal(buf, np.transpose(w["qkv"][steps - 3:steps], (1, 2, 0)))


def test_decode_batched_sequences_independent(ctx):
    steps, B = 4, 5
    w = W.dn_decode_workload(steps, B, seed=8)
    print("case: dn decode B=5 steps=4", flush=True)
    dev = DnDevice(ctx, w, steps, B)
    for t in range(steps):
        dev.step(t)
    ref, Sref = oracle_run(w, steps, B)
    assert np.abs(dev.outputs() - ref).max() <= TOL
    assert np.abs(dev.final_state() - Sref).max() <= TOL


@pytest.mark.parametrize("batch", [1, 3])
def test_decode_block_size_invariance_and_determinism(ctx, batch):
    """256/512/1024-thread workgroups give bit-identical results, run after run."""
    steps = 3
    w = W.dn_decode_workload(steps, batch, seed=21)
    results = []
    for threads in [256, 512, 1024, 1024]:
        print(f"case: dn decode threads={threads} B={batch}", flush=True)
        ctx.set_option(M.QM_OPT_DN_DECODE_THREADS, threads)
        dev = DnDevice(ctx, w, steps, batch)
        for t in range(steps):
            dev.step(t)
        results.append((dev.outputs(), dev.final_state()))
    ctx.set_option(M.QM_OPT_DN_DECODE_THREADS, 0)
    for o, s in results[1:]:
        assert np.array_equal(o, results[0][0]) and np.array_equal(s, results[0][1])


def test_decode_graph_replay_matches_eager(ctx):
    """A captured step replayed several times equals the same steps run eagerly."""
    w = W.dn_decode_workload(1, 1, seed=5)
    ctx.reserve(max_batch=8)
    eager = DnDevice(ctx, w, 1, 1)
    graphed = DnDevice(ctx, w, 1, 1)
    ctx.graph_begin()
    graphed.step(0)
    g = ctx.graph_end()
    for rep in range(4):
        print(f"case: dn decode graph replay {rep}", flush=True)
        eager.step(0)
        g.launch()
        ctx.sync()
        assert np.array_equal(eager.outputs(), graphed.outputs())
        assert np.array_equal(eager.final_state(), graphed.final_state())
    g.close()
