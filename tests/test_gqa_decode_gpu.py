"""GPU parity: GQA decode step (qm_gqa_decode) vs the CPU oracle.

The oracle restates gemv.rs:927-1011 on an f32 cache in the reference's
[seq][kv_head][dim] layout, filled with the f16 cache values (exact), with
the appended row rounded to f16 as the MI355X cache stores it.  Bar:
max-abs <= 1e-3 on the gated output.
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


def run_gpu(ctx, w, positions, rope_rows, chunk=0, pos_array=True):
    """pos_array=False passes no per-sequence positions (every sequence at
    max(positions), the batch-1 form)."""
    B = w["q_gate"].shape[0]
    cos, sin = M.rope_table(rope_rows)
    d = {k: ctx.upload(w[k]) for k in ["q_gate", "k_new", "v_new", "q_norm", "k_norm", "k_cache", "v_cache"]}
    rc, rs = ctx.upload(cos), ctx.upload(sin)
    pos_dev = ctx.upload(np.asarray(positions, np.int32)) if pos_array else None
    out = ctx.alloc(B * 16 * 256 * 4)
    ctx.set_option(M.QM_OPT_GQA_DECODE_CHUNK, chunk)
    try:
        ctx.gqa_decode(B, d["q_gate"], d["k_new"], d["v_new"], d["q_norm"], d["k_norm"], rc, rs,
                       rope_rows, pos_dev, int(max(positions)), d["k_cache"], d["v_cache"], w["cap"], out)
    finally:
        ctx.set_option(M.QM_OPT_GQA_DECODE_CHUNK, 0)
    o = ctx.download(out, (B, 16, 256), np.float32)
    kc = ctx.download(d["k_cache"], w["k_cache"].shape, np.uint16)
    vc = ctx.download(d["v_cache"], w["v_cache"].shape, np.uint16)
    return o, kc, vc


def run_oracle(w, positions, rope_rows):
    cfg = O.config()
    cos, sin = O.rope_table(rope_rows)
    B = w["q_gate"].shape[0]
    outs, krows, vrows = [], [], []
    for b in range(B):
        p = positions[b]
        K = np.ascontiguousarray(np.transpose(W.f16_value(w["k_cache"][b, :, :p + 1]), (1, 0, 2)))
        V = np.ascontiguousarray(np.transpose(W.f16_value(w["v_cache"][b, :, :p + 1]), (1, 0, 2)))
        o = O.attn_decode_step(cfg, w["q_gate"][b].ravel(), w["k_new"][b].ravel(), w["v_new"][b].ravel(),
                               w["q_norm"], w["k_norm"], cos, sin, K, V, p, round_kv_f16=True, nthreads=8)
        outs.append(o.reshape(16, 256))
        krows.append(K[p])
        vrows.append(V[p])
    return np.stack(outs), krows, vrows


def test_decode_pos4096_batch1(ctx):
    """One step at position 4096 (4097 keys), f16 cache."""
    w = W.gqa_decode_workload(4096, 1, seed=1)
    print("case: gqa decode B=1 pos=4096", flush=True)
    got, kc, vc = run_gpu(ctx, w, [4096], 4097)
    ref, krows, vrows = run_oracle(w, [4096], 4097)
    err = np.abs(got - ref).max()
    print(f"max|dout|={err:.3e}")
    assert err <= TOL
    # appended rows: f16 of the normed+roped k (within one f16 step) and of v (exact)
    kgot = W.f16_value(kc[0, :, 4096])
    assert np.all(np.abs(kgot - krows[0]) <= np.abs(krows[0]) * 2 ** -10 + 1e-7)
    assert np.array_equal(W.f16_value(vc[0, :, 4096]), vrows[0])


def test_decode_ragged_positions(ctx):
    """Sequences at different positions in one batch (pos_dev)."""
    positions = [0, 100, 2049, 777]
    w = W.gqa_decode_workload(2049, 4, cap=2100, seed=2)
    print("case: gqa decode ragged", positions, flush=True)
    got, _, _ = run_gpu(ctx, w, positions, 4096)
    ref, _, _ = run_oracle(w, positions, 4096)
    print(f"max|dout|={np.abs(got - ref).max():.3e}")
    assert np.abs(got - ref).max() <= TOL


@pytest.mark.parametrize("chunk", [0, 64, 192])
def test_decode_rows_past_the_end_never_reach_the_output(ctx, chunk):
    """Cache rows past a sequence's position may never have been written:
    here they hold f16 NaN and Inf (K and V), in the same rounds as valid keys
    and in whole rounds and splits past the end.  The outputs stay finite and
    equal the oracle's, which reads rows 0..pos only."""
    positions = [37, 1500, 64, 911]
    w = W.gqa_decode_workload(1500, 4, cap=1600, seed=21)
    for b, p in enumerate(positions):
        w["k_cache"][b, :, p + 1:] = np.uint16(0x7E00)            # NaN
        w["v_cache"][b, :, p + 1:] = np.uint16(0x7C00 if b % 2 else 0x7E00)   # +Inf / NaN
    print(f"case: gqa decode NaN/Inf past the end chunk={chunk}", positions, flush=True)
    got, _, _ = run_gpu(ctx, w, positions, 1501, chunk=chunk)
    ref, _, _ = run_oracle(w, positions, 1501)
    assert np.isfinite(got).all()
    print(f"max|dout|={np.abs(got - ref).max():.3e}")
    assert np.abs(got - ref).max() <= TOL


@pytest.mark.parametrize("chunk", [64, 128, 192, 1024, 4160])  # 128: eight waves; 4160: one split, no merge kernel
def test_decode_chunk_invariance(ctx, chunk):
    w = W.gqa_decode_workload(3000, 2, seed=3)
    print(f"case: gqa decode chunk={chunk}", flush=True)
    got, _, _ = run_gpu(ctx, w, [3000, 3000], 3001, chunk=chunk)
    ref, _, _ = run_oracle(w, [3000, 3000], 3001)
    assert np.abs(got - ref).max() <= TOL


@pytest.mark.parametrize("max_pos", [5000, 6000, 7000, 8000])
def test_decode_waves_per_split(ctx, max_pos):
    """Automatic splits of 80, 96, 112 and 128 keys at these lengths run five
    to eight waves per split workgroup (one 16-key round each).  The second
    sequence ends inside a split, so some waves there have no round."""
    positions = [max_pos, max_pos // 3 + 5]
    w = W.gqa_decode_workload(max_pos, 2, seed=31 + max_pos)
    print(f"case: gqa decode waves per split, positions {positions}", flush=True)
    got, _, _ = run_gpu(ctx, w, positions, max_pos + 1)
    ref, _, _ = run_oracle(w, positions, max_pos + 1)
    print(f"max|dout|={np.abs(got - ref).max():.3e}")
    assert np.abs(got - ref).max() <= TOL
    # batch 1 without a position array (the RoPE rows and the appended row
    # are loaded with the q row, ahead of the first round)
    w1 = W.gqa_decode_workload(max_pos, 1, seed=41 + max_pos)
    print(f"case: gqa decode waves per split, batch 1 at {max_pos}, no position array", flush=True)
    got, kc, _ = run_gpu(ctx, w1, [max_pos], max_pos + 1, pos_array=False)
    ref, krows, _ = run_oracle(w1, [max_pos], max_pos + 1)
    print(f"max|dout|={np.abs(got - ref).max():.3e}")
    assert np.abs(got - ref).max() <= TOL
    kgot = W.f16_value(kc[0, :, max_pos])
    assert np.all(np.abs(kgot - krows[0]) <= np.abs(krows[0]) * 2 ** -10 + 1e-7)


def test_decode_many_splits_ragged(ctx):
    """79 splits per sequence (more than one 64-split pass of the merge), and a
    short sequence whose splits past its end are empty (m = -inf)."""
    positions = [5000, 70]
    w = W.gqa_decode_workload(5000, 2, seed=11)
    print("case: gqa decode chunk=64 ragged", positions, flush=True)
    got, _, _ = run_gpu(ctx, w, positions, 5001, chunk=64)
    ref, _, _ = run_oracle(w, positions, 5001)
    print(f"max|dout|={np.abs(got - ref).max():.3e}")
    assert np.abs(got - ref).max() <= TOL


@pytest.mark.parametrize("positions", [[5000, 70, 4351, 640], [63, 64, 4095, 1000]])
def test_decode_multi_round_splits_ragged(ctx, positions):
    """192-key splits (three 64-key rounds of the four waves each): ragged
    lengths whose ends fall in different splits and rounds, appends at round
    edges (63, 64, 4095), and sequences so short that most splits are empty."""
    w = W.gqa_decode_workload(5000, len(positions), seed=13)
    print("case: gqa decode chunk=192 ragged", positions, flush=True)
    got, kc, vc = run_gpu(ctx, w, positions, 5001, chunk=192)
    ref, krows, vrows = run_oracle(w, positions, 5001)
    print(f"max|dout|={np.abs(got - ref).max():.3e}")
    assert np.abs(got - ref).max() <= TOL
    for b, p in enumerate(positions):              # each sequence's row appended by the split that owns it
        kgot, vgot = W.f16_value(kc[b, :, p]), W.f16_value(vc[b, :, p])
        assert np.all(np.abs(kgot - krows[b]) <= np.abs(krows[b]) * 2 ** -10 + 1e-7)
        assert np.array_equal(vgot, vrows[b])


def test_decode_range_errors(ctx):
    w = W.gqa_decode_workload(16, 1, cap=17, seed=4)
    cos, sin = M.rope_table(16)
    d = {k: ctx.upload(w[k]) for k in ["q_gate", "k_new", "v_new", "q_norm", "k_norm", "k_cache", "v_cache"]}
    rc, rs = ctx.upload(cos), ctx.upload(sin)
    out = ctx.alloc(16 * 256 * 4)
    with pytest.raises(M.MixerError) as e:      # position 16 with a 16-row table
        ctx.gqa_decode(1, d["q_gate"], d["k_new"], d["v_new"], d["q_norm"], d["k_norm"], rc, rs, 16,
                       None, 16, d["k_cache"], d["v_cache"], 17, out)
    assert e.value.code == 5
    with pytest.raises(M.MixerError) as e:      # position 17 with capacity 17
        ctx.gqa_decode(1, d["q_gate"], d["k_new"], d["v_new"], d["q_norm"], d["k_norm"], rc, rs, 64,
                       None, 17, d["k_cache"], d["v_cache"], 17, out)
    assert e.value.code == 6
    with pytest.raises(M.MixerError) as e:      # q_gate 8 bytes off 16-byte alignment
        ctx.gqa_decode(1, d["q_gate"].offset(8), d["k_new"], d["v_new"], d["q_norm"], d["k_norm"], rc, rs, 16,
                       None, 4, d["k_cache"], d["v_cache"], 17, out)
    assert e.value.code == 3                    # QM_ERR_INVALID_ARG
    with pytest.raises(M.MixerError) as e:      # same for the prefill entry
        ctx.gqa_prefill(4, d["q_gate"], d["k_new"], d["v_new"], d["q_norm"].offset(2), d["k_norm"], rc, rs, 16,
                        d["k_cache"], d["v_cache"], 17, out)
    assert e.value.code == 3                    # QM_ERR_INVALID_ARG


def test_decode_graph_replay_matches_eager(ctx):
    """One captured decode step (split + merge) replayed several times, with
    eager launches and synchronisations in between, matches the eager step
    bit for bit on every replay (the step is idempotent: it rewrites cache row
    `pos` and reads rows 0..pos)."""
    pos = 300
    w = W.gqa_decode_workload(pos, 2, seed=9)
    cos, sin = M.rope_table(pos + 1)
    d = {k: ctx.upload(w[k]) for k in ["q_gate", "k_new", "v_new", "q_norm", "k_norm", "k_cache", "v_cache"]}
    rc, rs = ctx.upload(cos), ctx.upload(sin)
    out_e, out_g = ctx.alloc(2 * 16 * 256 * 4), ctx.alloc(2 * 16 * 256 * 4)
    ctx.reserve(max_batch=2, max_kv_len=pos + 1)

    def step(out):
        ctx.gqa_decode(2, d["q_gate"], d["k_new"], d["v_new"], d["q_norm"], d["k_norm"], rc, rs, pos + 1,
                       None, pos, d["k_cache"], d["v_cache"], w["cap"], out)

    print("case: gqa decode graph replay (eager reference)", flush=True)
    step(out_e)
    ref = ctx.download(out_e, (2, 16 * 256), np.float32)
    ctx.graph_begin()
    step(out_g)
    g = ctx.graph_end()
    for rep in range(4):
        print(f"case: gqa decode graph replay {rep}", flush=True)
        ctx.fill_normal(out_g, M.QM_F32, 2 * 16 * 256, 0.0, 1.0, seed=rep)   # poison between replays
        g.launch()
        ctx.sync()
        assert np.array_equal(ctx.download(out_g, (2, 16 * 256), np.float32), ref)
        step(out_e)                                                           # eager work in between
        ctx.sync()


def test_graph_survives_workspace_growth():
    """A graph captured on a context whose workspace later grows (an eager call
    at a longer KV length, no qm_reserve) still replays to the same result:
    the grown-out-of workspace stays allocated while the context lives."""
    pos_small, pos_big = 300, 4000
    w = W.gqa_decode_workload(pos_big, 2, seed=12)
    cos, sin = M.rope_table(pos_big + 1)
    with M.Context(0) as c:                    # fresh context: workspace starts empty
        d = {k: c.upload(w[k]) for k in ["q_gate", "k_new", "v_new", "q_norm", "k_norm", "k_cache", "v_cache"]}
        rc, rs = c.upload(cos), c.upload(sin)
        out_e, out_g = c.alloc(2 * 16 * 256 * 4), c.alloc(2 * 16 * 256 * 4)
        c.set_option(M.QM_OPT_GQA_DECODE_CHUNK, 64)   # many splits: the partials grow with the length

        def step(pos, out):
            c.gqa_decode(2, d["q_gate"], d["k_new"], d["v_new"], d["q_norm"], d["k_norm"], rc, rs, pos_big + 1,
                         None, pos, d["k_cache"], d["v_cache"], w["cap"], out)

        print("case: gqa decode graph, then workspace growth", flush=True)
        step(pos_small, out_e)                  # sizes the workspace for pos 300
        ref = c.download(out_e, (2, 16 * 256), np.float32)
        c.graph_begin()
        step(pos_small, out_g)
        g = c.graph_end()
        step(pos_big, out_e)                    # grows the workspace (79 splits vs 5)
        c.sync()
        for rep in range(3):
            c.fill_normal(out_g, M.QM_F32, 2 * 16 * 256, 0.0, 1.0, seed=rep)
            g.launch()
            c.sync()
            assert np.array_equal(c.download(out_g, (2, 16 * 256), np.float32), ref)
            step(pos_big, out_e)
            c.sync()
        g.close()
