#!/usr/bin/env python3
"""Token-mixer benchmark on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload NAME]

Workloads (synthetic, seeded; inputs resident in HBM before timing):
  stack       32-layer hybrid mixer stack (3x DeltaNet + 1x GQA, x8) in batched
              decode: 64 sequences at context 32768, one step = one token per
              sequence through all 32 mixers.  Default; the headline line.
  dn_decode   one DeltaNet layer, batch 1, one step = one token.
  gqa_decode  one GQA layer, batch 1, one step at position 4096.
  dn_prefill  one DeltaNet layer, chunked prefill of 4096 tokens (bf16 in,
              fp32 state), one step = one prefill call.
  gqa_prefill one GQA layer, causal prefill of 8192 tokens (bf16 in, f16 KV
              cache written), one step = one prefill call.
--gqa-chunk N sets the keys per GQA decode split workgroup (default: the
library's choice).
Prints one JSON line with throughput, the dominant kernel's roofline
position (average launch time from HIP events on the launch stream) and the
CPU oracle timed on this host on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
HBM_PEAK = 8.0e12          # MI355X HBM3E, bytes/s
MFMA_BF16_PEAK = 2.5e15    # MI355X dense bf16/f16 MFMA, flop/s
N_DN, N_GQA = 24, 8        # 3x DeltaNet + 1x GQA, repeated 8 times (config.rs:44-50)
# the sources of the GQA decode kernels whose rocprofv3 traffic is stored
GQA_DECODE_SOURCES = ("qora-llm-4b_amd/csrc/gqa_decode.hip", "qora-llm-4b_amd/csrc/qm_gqa_common.h")


def _load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


M = _load("qora_mixer", ROOT / "qora-llm-4b_amd" / "qora_mixer.py")
W = _load("qora_workloads", ROOT / "qora-llm-4b_amd" / "workloads.py")


def host_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


# ----------------------------------------------------------------------------
# algorithmic bytes
def dn_decode_bytes(batch: int) -> int:
    """State read + write plus the per-token vectors, per launch."""
    state = 2 * 32 * 128 * 128 * 4
    vec = (8192 + 32 + 32 + 4096 + 4096) * 4          # act q|k|v, a, b, z, out
    params = (32 + 32) * 4 + 128 * 2                   # A_log, dt_bias, norm weight
    return batch * (state + vec) + params


def gqa_decode_bytes(batch: int, length: int) -> int:
    """K and V rows 0..len-1 read, new row written, per-token vectors."""
    kv = 2 * 4 * length * 256 * 2
    vec = (16 * 512 + 2 * 4 * 256 + 16 * 256) * 4
    rope = 2 * 32 * 4
    return batch * (kv + vec + rope) + 2 * 256 * 2


def dn_prefill_flops(T: int, C: int = 64) -> int:
    """Chunked-form flops per layer: per head and chunk 5 C x C x d products
    (KK^T, QK^T, W, U~, P U~) and 3 C x d x d products (W S^T, Q~ S^T,
    U^T K~); the triangular solve is not counted."""
    d, H = 128, 32
    nc = -(-T // C)
    return H * nc * (5 * 2 * C * C * d + 3 * 2 * C * d * d)


def gqa_prefill_flops(S: int) -> int:
    """QK^T and PV over the causal triangle: 2 products x 2 flop x D x H x S(S+1)/2."""
    return 2 * 2 * 256 * 16 * S * (S + 1) // 2


# ----------------------------------------------------------------------------
class Timer:
    """HIP events on the launch stream around every launch of one kernel."""

    def __init__(self, ctx):
        self.ctx = ctx
        self.pairs = []

    def wrap(self, fn):
        a, b = self.ctx.event(), self.ctx.event()
        a.record()
        fn()
        b.record()
        self.pairs.append((a, b))

    def mean_ms(self):
        return float(np.mean([a.elapsed_ms(b) for a, b in self.pairs])) if self.pairs else float("nan")


def run_stack(args, ctx):
    B, ctx0 = 64, 32768
    K, Wm = args.steps, args.warmup
    total_steps = K + Wm
    cap = ctx0 + total_steps
    rope_rows = cap + 1
    rng = np.random.default_rng(4)
    seed = [1000]

    def fill(buf, dtype, count, std, mean=0.0):
        seed[0] += 1
        ctx.fill_normal(buf, dtype, count, mean, std, seed[0])

    # per-layer parameters (host generated, tiny)
    dn_par = []
    for _ in range(N_DN):
        p = W.dn_params(rng)
        dn_par.append({k: ctx.upload(p[k]) for k in ["a_log", "dt_bias", "norm_w"]})
    gqa_par = []
    for _ in range(N_GQA):
        gqa_par.append({
            "q_norm": ctx.upload(W.f16_bits(0.1 * rng.standard_normal(256, dtype=np.float32))),
            "k_norm": ctx.upload(W.f16_bits(0.1 * rng.standard_normal(256, dtype=np.float32))),
        })
    cos, sin = M.rope_table(rope_rows)
    rc, rs = ctx.upload(cos), ctx.upload(sin)

    # state, caches, per-step inputs: all in HBM
    S_LAYER = B * 32 * 128 * 128
    states = [ctx.alloc(S_LAYER * 4) for _ in range(N_DN)]
    for s in states:
        fill(s, M.QM_F32, S_LAYER, 0.02)
    KV_LAYER = B * 4 * cap * 256
    kcs = [ctx.alloc(KV_LAYER * 2) for _ in range(N_GQA)]
    vcs = [ctx.alloc(KV_LAYER * 2) for _ in range(N_GQA)]
    for buf in kcs + vcs:
        fill(buf, M.QM_F16, KV_LAYER, 1.0)
    DN_IN = B * (8192 + 32 + 32 + 4096)
    dn_in = ctx.alloc(total_steps * N_DN * DN_IN * 4)
    fill(dn_in, M.QM_F32, total_steps * N_DN * DN_IN, 1.0)
    GQA_IN = B * (16 * 512 + 2 * 4 * 256)
    gqa_in = ctx.alloc(total_steps * N_GQA * GQA_IN * 4)
    fill(gqa_in, M.QM_F32, total_steps * N_GQA * GQA_IN, 1.0)
    dn_out = ctx.alloc(B * 4096 * 4)
    gqa_out = ctx.alloc(B * 16 * 256 * 4)
    ctx.reserve(max_batch=B, max_kv_len=cap)
    ctx.sync()

    dn_timer, gqa_timer = Timer(ctx), Timer(ctx)

    def step(s, timed):
        pos = ctx0 + s
        li_dn = li_gqa = 0
        for layer in range(32):
            if layer % 4 != 3:
                base = dn_in.offset(((s * N_DN + li_dn) * DN_IN) * 4)
                qkv = base
                a = base + B * 8192 * 4
                b = a + B * 32 * 4
                z = b + B * 32 * 4
                p = dn_par[li_dn]
                call = lambda: ctx.deltanet_decode(B, M.QM_DN_POSTACT, qkv, None, None, a, b,
                                                   p["a_log"], p["dt_bias"], z, p["norm_w"],
                                                   states[li_dn], dn_out)
                dn_timer.wrap(call) if timed else call()
                li_dn += 1
            else:
                base = gqa_in.offset(((s * N_GQA + li_gqa) * GQA_IN) * 4)
                qg = base
                kn = qg + B * 16 * 512 * 4
                vn = kn + B * 4 * 256 * 4
                p = gqa_par[li_gqa]
                call = lambda: ctx.gqa_decode(B, qg, kn, vn, p["q_norm"], p["k_norm"], rc, rs,
                                              rope_rows, None, pos, kcs[li_gqa], vcs[li_gqa], cap,
                                              gqa_out)
                gqa_timer.wrap(call) if timed else call()
                li_gqa += 1

    for s in range(Wm):
        step(s, False)
    ctx.sync()
    t0 = ctx.event()
    t1 = ctx.event()
    wall0 = time.perf_counter()
    t0.record()
    for s in range(Wm, Wm + K):
        step(s, True)
    t1.record()
    ctx.sync()
    wall = time.perf_counter() - wall0
    total_ms = t0.elapsed_ms(t1)

    # GQA kernel: average length over the timed steps
    mean_len = ctx0 + Wm + (K - 1) / 2.0 + 1
    gqa_ms = gqa_timer.mean_ms()
    dn_ms = dn_timer.mean_ms()
    gqa_bytes = gqa_decode_bytes(B, int(round(mean_len)))
    dn_bytes = dn_decode_bytes(B)
    step_bytes = N_DN * dn_bytes + N_GQA * gqa_bytes
    res = {
        "tokens": B * K, "total_ms": total_ms, "wall_s": wall,
        "dominant": "qm_gqa_decode_split+merge",
        "roofline": {"bound": "hbm", "achieved": gqa_bytes / (gqa_ms * 1e-3), "peak": HBM_PEAK,
                     "unit": "GB/s", "kernel_ms": gqa_ms, "bytes_per_launch": gqa_bytes},
        "kernels": {
            "qm_gqa_decode_split+merge": {"avg_ms": gqa_ms, "bytes": gqa_bytes,
                              "GB_s": gqa_bytes / gqa_ms / 1e6, "frac_hbm": gqa_bytes / (gqa_ms * 1e-3) / HBM_PEAK},
            "qm_dn_decode_t256": {"avg_ms": dn_ms, "bytes": dn_bytes,
                                "GB_s": dn_bytes / dn_ms / 1e6, "frac_hbm": dn_bytes / (dn_ms * 1e-3) / HBM_PEAK},
        },
        "step_frac_hbm": step_bytes * K / (total_ms * 1e-3) / HBM_PEAK,
        "config": {"workload": "hybrid mixer stack decode: 32 layers (24 DeltaNet + 8 GQA), "
                               "64 sequences, context 32768, f16 KV, fp32 state",
                   "batch": B, "context": ctx0, "layers": 32, "seq_len": ctx0, "global_batch": B,
                   "parallelism": "single GPU"},
    }
    return res


def run_dn_decode(args, ctx):
    K, Wm = args.steps, args.warmup
    w = W.dn_decode_workload(K + Wm, 1, seed=0)
    up = ctx.upload
    qkv, a, b, z = up(w["qkv"]), up(w["a"]), up(w["b"]), up(w["z"])
    a_log, dt_bias, norm_w = up(w["a_log"]), up(w["dt_bias"]), up(w["norm_w"])
    state = up(w["state0"])
    out = ctx.alloc((K + Wm) * 4096 * 4)
    ctx.reserve(max_batch=1)

    def step(t):
        ctx.deltanet_decode(1, M.QM_DN_POSTACT, qkv.offset(t * 8192 * 4), None, None,
                            a.offset(t * 32 * 4), b.offset(t * 32 * 4), a_log, dt_bias,
                            z.offset(t * 4096 * 4), norm_w, state, out.offset(t * 4096 * 4))

    for t in range(Wm):
        step(t)
    # the timed steps run from one captured graph (one launch per step inside)
    ctx.graph_begin()
    for t in range(Wm, Wm + K):
        step(t)
    g = ctx.graph_end()
    ctx.sync()
    t0, t1 = ctx.event(), ctx.event()
    wall0 = time.perf_counter()
    t0.record()
    g.launch()
    t1.record()
    ctx.sync()
    wall = time.perf_counter() - wall0
    total_ms = t0.elapsed_ms(t1)
    # per-launch device time: the graph runs the K launches back to back, so
    # events around it over K give the average launch duration (events around
    # single eager launches at batch 1 measure host submission gaps instead)
    k_ms = total_ms / K
    tm = Timer(ctx)
    for t in range(min(K, 64)):
        tm.wrap(lambda: step(Wm + t))
    ctx.sync()
    nbytes = dn_decode_bytes(1)
    # Cold variant: the 2 MiB state stays in L2 / the 256 MB MALL across the
    # steps above.  Here step t updates state t mod NS of NS = 256 distinct
    # states (512 MiB), so each launch finds its state evicted by the 255
    # launches since its last use.
    NS = 256
    states = ctx.alloc(NS * 32 * 128 * 128 * 4)
    ctx.fill_normal(states, M.QM_F32, NS * 32 * 128 * 128, 0.0, 0.02, 40)

    def step_cold(t, i):
        ctx.deltanet_decode(1, M.QM_DN_POSTACT, qkv.offset(t * 8192 * 4), None, None,
                            a.offset(t * 32 * 4), b.offset(t * 32 * 4), a_log, dt_bias,
                            z.offset(t * 4096 * 4), norm_w, states.offset((i % NS) * 32 * 128 * 128 * 4),
                            out.offset(t * 4096 * 4))

    ctx.graph_begin()
    for i in range(K):
        step_cold(Wm + i, i)
    gc_ = ctx.graph_end()
    gc_.launch()                          # warm-up replay: every state touched once
    ctx.sync()
    c0, c1 = ctx.event(), ctx.event()
    c0.record()
    gc_.launch()
    c1.record()
    ctx.sync()
    cold_ms = c0.elapsed_ms(c1) / K
    gc_.close()
    states.close()
    return {
        "tokens": K, "total_ms": total_ms, "wall_s": wall, "dominant": "qm_dn_decode_t512",
        "roofline": {"bound": "hbm", "achieved": nbytes / (k_ms * 1e-3), "peak": HBM_PEAK,
                     "unit": "GB/s", "kernel_ms": k_ms, "bytes_per_launch": nbytes},
        "eager_event_ms_per_launch": tm.mean_ms(),
        "cold": {"ms_per_launch": cold_ms, "frac": nbytes / (cold_ms * 1e-3) / HBM_PEAK,
                 "note": f"graph of {K} steps rotating over {NS} states ({NS * 2} MiB)"},
        "config": {"workload": "DeltaNet decode, 1 layer, batch 1, 16 qk / 32 v heads x 128, fp32 state",
                   "batch": 1, "seq_len": K, "global_batch": 1, "parallelism": "single GPU"},
    }


def run_gqa_decode(args, ctx):
    K, Wm = args.steps, args.warmup
    pos = 4096
    w = W.gqa_decode_workload(pos, 1, seed=1)
    cos, sin = M.rope_table(pos + 1)
    d = {k: ctx.upload(w[k]) for k in ["q_gate", "k_new", "v_new", "q_norm", "k_norm", "k_cache", "v_cache"]}
    rc, rs = ctx.upload(cos), ctx.upload(sin)
    out = ctx.alloc(16 * 256 * 4)
    ctx.reserve(max_batch=1, max_kv_len=pos + 1)

    def step():
        ctx.gqa_decode(1, d["q_gate"], d["k_new"], d["v_new"], d["q_norm"], d["k_norm"], rc, rs,
                       pos + 1, None, pos, d["k_cache"], d["v_cache"], w["cap"], out)

    for _ in range(Wm):
        step()
    # the timed steps run from one captured graph (split + merge per step);
    # each step rewrites cache row `pos` and reads rows 0..pos
    ctx.graph_begin()
    for _ in range(K):
        step()
    g = ctx.graph_end()
    ctx.sync()
    t0, t1 = ctx.event(), ctx.event()
    wall0 = time.perf_counter()
    t0.record()
    g.launch()
    t1.record()
    ctx.sync()
    wall = time.perf_counter() - wall0
    total_ms = t0.elapsed_ms(t1)
    k_ms = total_ms / K                      # device time per split + merge pair
    tm = Timer(ctx)
    for _ in range(min(K, 64)):
        tm.wrap(step)
    ctx.sync()
    nbytes = gqa_decode_bytes(1, pos + 1)
    # Cold variant: one 16 MiB cache stays resident in the 256 MB MALL across
    # the steps above.  Here step i reads cache i mod NC of NC = 40 distinct
    # caches (~670 MB), so each launch finds its cache evicted by the 39
    # launches since its last use.
    NC = 40
    cache_elems = 4 * w["cap"] * 256
    kcs, vcs = ctx.alloc(NC * cache_elems * 2), ctx.alloc(NC * cache_elems * 2)
    ctx.fill_normal(kcs, M.QM_F16, NC * cache_elems, 0.0, 1.0, 41)
    ctx.fill_normal(vcs, M.QM_F16, NC * cache_elems, 0.0, 1.0, 42)

    def step_cold(i):
        j = (i % NC) * cache_elems * 2
        ctx.gqa_decode(1, d["q_gate"], d["k_new"], d["v_new"], d["q_norm"], d["k_norm"], rc, rs,
                       pos + 1, None, pos, kcs.offset(j), vcs.offset(j), w["cap"], out)

    ctx.graph_begin()
    for i in range(K):
        step_cold(i)
    gc_ = ctx.graph_end()
    gc_.launch()                          # warm-up replay
    ctx.sync()
    c0, c1 = ctx.event(), ctx.event()
    c0.record()
    gc_.launch()
    c1.record()
    ctx.sync()
    cold_ms = c0.elapsed_ms(c1) / K
    gc_.close()
    kcs.close()
    vcs.close()
    return {
        "tokens": K, "total_ms": total_ms, "wall_s": wall, "dominant": "qm_gqa_decode_split+merge",
        "roofline": {"bound": "hbm", "achieved": nbytes / (k_ms * 1e-3), "peak": HBM_PEAK,
                     "unit": "GB/s", "kernel_ms": k_ms, "bytes_per_launch": nbytes},
        "eager_event_ms_per_launch": tm.mean_ms(),
        "cold": {"ms_per_launch": cold_ms, "frac": nbytes / (cold_ms * 1e-3) / HBM_PEAK,
                 "note": f"graph of {K} steps rotating over {NC} caches ({NC * 2 * cache_elems * 2 / 2**20:.0f} MiB)"},
        "config": {"workload": "GQA decode, 1 layer, batch 1, 16q/4kv x 256, position 4096, f16 KV",
                   "batch": 1, "seq_len": pos + 1, "global_batch": 1, "parallelism": "single GPU"},
    }


def run_dn_prefill(args, ctx):
    K, Wm = args.steps, args.warmup
    T = 4096
    w = W.dn_prefill_workload(T, seed=2)
    up = ctx.upload
    d = {k: up(w[k]) for k in ["qkv", "conv_w", "a", "b", "a_log", "dt_bias", "z", "norm_w"]}
    state, buf = up(w["state0"]), up(w["conv_buf0"])
    out = ctx.alloc(T * 4096 * 2)
    ctx.reserve(max_batch=1, max_prefill_tokens=T)

    def step():
        ctx.deltanet_prefill(T, d["qkv"], buf, d["conv_w"], d["a"], d["b"], d["a_log"], d["dt_bias"],
                             d["z"], d["norm_w"], state, out)

    for _ in range(Wm):
        step()
    ctx.sync()
    tm = Timer(ctx)
    t0, t1 = ctx.event(), ctx.event()
    wall0 = time.perf_counter()
    t0.record()
    for _ in range(K):
        tm.wrap(step)
    t1.record()
    ctx.sync()
    wall = time.perf_counter() - wall0
    total_ms = t0.elapsed_ms(t1)
    k_ms = tm.mean_ms()
    flops = dn_prefill_flops(T)
    return {
        "tokens": K * T, "total_ms": total_ms, "wall_s": wall,
        "dominant": "qm_deltanet_prefill (chunk+scan+out)",
        "roofline": {"bound": "mfma", "achieved": flops / (k_ms * 1e-3), "peak": MFMA_BF16_PEAK,
                     "unit": "TFLOP/s", "kernel_ms": k_ms, "flops_per_launch": flops},
        "config": {"workload": "DeltaNet chunked prefill, 1 layer, batch 1, seq 4096, chunk 64, "
                               "bf16 in, fp32 state", "batch": 1, "seq_len": T, "global_batch": 1,
                   "parallelism": "single GPU"},
    }


def run_gqa_prefill(args, ctx):
    K, Wm = args.steps, args.warmup
    S = 8192
    w = W.gqa_prefill_workload(S, seed=3)
    cos, sin = M.rope_table(S)
    d = {k: ctx.upload(w[k]) for k in ["q_gate", "k", "v", "q_norm", "k_norm"]}
    rc, rs = ctx.upload(cos), ctx.upload(sin)
    kc, vc = ctx.alloc(4 * S * 256 * 2), ctx.alloc(4 * S * 256 * 2)
    out = ctx.alloc(S * 16 * 256 * 2)
    ctx.reserve(max_batch=1, max_prefill_tokens=S)

    def step():
        ctx.gqa_prefill(S, d["q_gate"], d["k"], d["v"], d["q_norm"], d["k_norm"], rc, rs, S, kc, vc, S, out)

    for _ in range(Wm):
        step()
    ctx.sync()
    tm = Timer(ctx)
    t0, t1 = ctx.event(), ctx.event()
    wall0 = time.perf_counter()
    t0.record()
    for _ in range(K):
        tm.wrap(step)
    t1.record()
    ctx.sync()
    wall = time.perf_counter() - wall0
    total_ms = t0.elapsed_ms(t1)
    k_ms = tm.mean_ms()
    flops = gqa_prefill_flops(S)
    return {
        "tokens": K * S, "total_ms": total_ms, "wall_s": wall,
        "dominant": "qm_gqa_prefill (kv+attn)",
        "roofline": {"bound": "mfma", "achieved": flops / (k_ms * 1e-3), "peak": MFMA_BF16_PEAK,
                     "unit": "TFLOP/s", "kernel_ms": k_ms, "flops_per_launch": flops},
        "config": {"workload": "GQA causal prefill, 1 layer, batch 1, seq 8192, 16q/4kv x 256, "
                               "bf16 in, f16 KV cache out", "batch": 1, "seq_len": S,
                   "global_batch": 1, "parallelism": "single GPU"},
    }


# ----------------------------------------------------------------------------
# CPU baseline: the oracle (C restatement of the reference CPU path) on this host
CPU_SAMPLE_S = 10.0        # minimum seconds of CPU work per baseline sample


Q4_LAYER_PROJ = ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b", "out_proj",
                 "gate_proj", "up_proj", "down_proj")
Q4_LAYERS = 24   # DeltaNet layers of the 4B stack


def q4_gemv_bytes(k: int, n: int) -> int:
    """Algorithmic HBM bytes of one Q4 GEMV: codes, scales, x in, y out."""
    return k * n // 2 + k * (n // 32) * 2 + 4 * k + 4 * n


def q4_weight_bytes(k: int, n: int) -> int:
    return k * n // 2 + k * (n // 32) * 2


def run_q4_proj(args, ctx):
    """One decode token through the Q4 projections of the 24 DeltaNet layers,
    each layer with its own weights (1.52 GB, far beyond the 256 MB MALL, so
    every launch streams its weights from HBM).  Per layer, four launches:
      1. input RMSNorm + in_proj_qkv, in_proj_z, in_proj_a, in_proj_b;
      2. out_proj + residual;
      3. post-attention RMSNorm + gate_proj, up_proj + SiLU gate;
      4. down_proj + residual
    (gemv.rs:740-742,788-789,865,886-897; the mixer itself runs between 1
    and 2 and is measured by the other workloads)."""
    K, Wm = args.steps, args.warmup
    shapes = {nm: W.Q4_PROJ_SHAPES[nm] for nm in Q4_LAYER_PROJ}
    seed = [3000]

    def fill(buf, dtype, count, std, mean=0.0):
        ctx.fill_normal(buf, dtype, count, mean, std, seed[0])
        seed[0] += 1

    def weight(k, n):
        # the device layout directly (codes [n/T][k][T/2], scales [n/32][k]):
        # any byte is a valid pair of codes; scales ~ absmax/7 of N(0, 0.02) groups
        codes = ctx.alloc(k * n // 2)
        fill(codes, M.QM_F16, k * n // 4, 1.0)
        gscales = ctx.alloc(max(16, k * (n // 32) * 2))
        fill(gscales, M.QM_F16, k * (n // 32), 0.0012, 0.006)
        return codes, gscales

    layers = [{nm: weight(*shapes[nm]) for nm in Q4_LAYER_PROJ} for _ in range(Q4_LAYERS)]
    norms = ctx.alloc(2560 * 2)
    fill(norms, M.QM_F16, 2560, 0.1)
    h = ctx.alloc(2560 * 4)
    fill(h, M.QM_F32, 2560, 1.0)
    mixer_out = ctx.alloc(4096 * 4)
    fill(mixer_out, M.QM_F32, 4096, 1.0)
    ys = {nm: ctx.alloc(shapes[nm][1] * 4) for nm in ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b")}
    inter = ctx.alloc(9216 * 4)
    ctx.reserve(max_batch=1)
    timers = {kind: Timer(ctx) for kind in ("in", "out", "gate_up", "down")}

    def step(timed):
        for L in layers:
            calls = {
                "in": lambda: ctx.q4_gemv_multi(2560, h, [
                    (shapes[nm][1], L[nm][0], L[nm][1], ys[nm])
                    for nm in ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b")], norm_w=norms),
                "out": lambda: ctx.q4_gemv_multi(4096, mixer_out, [
                    (2560, L["out_proj"][0], L["out_proj"][1], h, h)]),
                "gate_up": lambda: ctx.q4_gate_up(2560, 9216, h, norms, *L["gate_proj"], *L["up_proj"], inter),
                "down": lambda: ctx.q4_gemv_multi(9216, inter, [
                    (2560, L["down_proj"][0], L["down_proj"][1], h, h)]),
            }
            for kind, call in calls.items():
                timers[kind].wrap(call) if timed else call()

    for _ in range(Wm):
        step(False)
    ctx.sync()
    t0, t1 = ctx.event(), ctx.event()
    wall0 = time.perf_counter()
    t0.record()
    for _ in range(K):
        step(True)
    t1.record()
    ctx.sync()
    wall = time.perf_counter() - wall0
    total_ms = t0.elapsed_ms(t1)
    graph_ms = float("nan")
    if not args.no_graph:
        # the same step captured once and replayed (no host launch cost)
        ctx.graph_begin()
        step(False)
        g = ctx.graph_end()
        g.launch()
        ctx.sync()
        g0, g1 = ctx.event(), ctx.event()
        g0.record()
        for _ in range(K):
            g.launch()
        g1.record()
        ctx.sync()
        graph_ms = g0.elapsed_ms(g1) / K
        g.close()
    wb = {nm: q4_weight_bytes(*shapes[nm]) for nm in Q4_LAYER_PROJ}
    kbytes = {   # weights + activations read + outputs written, per launch
        "in": sum(wb[nm] for nm in ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b"))
              + 2560 * 6 + 4 * (8192 + 4096 + 64),
        "out": wb["out_proj"] + 4096 * 4 + 2560 * 8,
        "gate_up": wb["gate_proj"] + wb["up_proj"] + 2560 * 6 + 9216 * 4,
        "down": wb["down_proj"] + 9216 * 4 + 2560 * 8,
    }
    names = {"in": "qm_q4_gemv (RMSNorm + in_proj_qkv/z/a/b)", "out": "qm_q4_gemv (out_proj + residual)",
             "gate_up": "qm_q4_gate_up (RMSNorm + gate/up + SiLU)", "down": "qm_q4_gemv (down_proj + residual)"}
    kernels = {names[kd]: {"avg_ms": timers[kd].mean_ms(), "bytes": kbytes[kd],
                           "GB_s": kbytes[kd] / timers[kd].mean_ms() / 1e6,
                           "frac_hbm": kbytes[kd] / (timers[kd].mean_ms() * 1e-3) / HBM_PEAK}
               for kd in timers}
    step_bytes = Q4_LAYERS * sum(kbytes.values())
    gu_ms = timers["gate_up"].mean_ms()
    return {
        "tokens": K, "total_ms": total_ms, "wall_s": wall,
        "dominant": names["gate_up"],
        "roofline": {"bound": "hbm", "achieved": kbytes["gate_up"] / (gu_ms * 1e-3), "peak": HBM_PEAK,
                     "kernel_ms": gu_ms, "bytes_per_launch": kbytes["gate_up"]},
        "kernels": kernels,
        "step_frac_hbm": step_bytes / (total_ms / K * 1e-3) / HBM_PEAK,
        "graph_ms_per_step": graph_ms,
        "graph_step_frac_hbm": step_bytes / (graph_ms * 1e-3) / HBM_PEAK,
        "config": {"workload": "Q4 decode projections of the 24 DeltaNet layers: input RMSNorm + "
                               "in_proj_qkv 2560x8192, in_proj_z 2560x4096, in_proj_a/b 2560x32; "
                               "out_proj 4096x2560 + residual; RMSNorm + gate/up 2560x9216 + SiLU; "
                               "down_proj 9216x2560 + residual; batch 1, one weight set per layer",
                   "batch": 1, "seq_len": 1, "global_batch": 1, "parallelism": "single GPU"},
    }


def run_q4_gemm(args, ctx):
    """The prefill form of a Q4 projection: in_proj_qkv (2560 x 8192) for a
    4096-token prompt on MFMA, f16 input rows (the RMSNormed hidden state),
    bf16 output (what the chunked DeltaNet prefill reads)."""
    K, Wm = args.steps, args.warmup
    m, (k, n) = 4096, W.Q4_PROJ_SHAPES["in_proj_qkv"]
    seed = [4000]

    def fill(buf, dtype, count, std, mean=0.0):
        ctx.fill_normal(buf, dtype, count, mean, std, seed[0])
        seed[0] += 1

    codes = ctx.alloc(k * n // 2)
    fill(codes, M.QM_F16, k * n // 4, 1.0)                # any byte is a valid pair of codes
    gscales = ctx.alloc(k * (n // 32) * 2)
    fill(gscales, M.QM_F16, k * (n // 32), 0.0012, 0.006)
    x = ctx.alloc(m * k * 2)
    fill(x, M.QM_F16, m * k, 1.0)
    y = ctx.alloc(m * n * 2)
    tm = Timer(ctx)

    def step():
        ctx.q4_gemm(m, k, n, x, codes, gscales, y_bf16=y)

    for _ in range(Wm):
        step()
    ctx.sync()
    t0, t1 = ctx.event(), ctx.event()
    wall0 = time.perf_counter()
    t0.record()
    for _ in range(K):
        tm.wrap(step)
    t1.record()
    ctx.sync()
    wall = time.perf_counter() - wall0
    flops = 2 * m * k * n
    k_ms = tm.mean_ms()
    return {
        "tokens": K * m, "total_ms": t0.elapsed_ms(t1), "wall_s": wall,
        "dominant": "qm_q4_gemm (in_proj_qkv, 4096 x 2560 x 8192)",
        "roofline": {"bound": "mfma", "achieved": flops / (k_ms * 1e-3), "peak": MFMA_BF16_PEAK,
                     "kernel_ms": k_ms, "flops_per_launch": flops},
        "config": {"workload": "Q4 prefill projection in_proj_qkv: 4096 tokens x 2560 -> 8192, f16 input, "
                               "Q4 weight dequantized to f16 on MFMA, bf16 output",
                   "batch": 1, "seq_len": m, "global_batch": 1, "parallelism": "single GPU"},
    }


LM_VOCAB, LM_HIDDEN = 248320, 2560


def lm_head_bytes(vocab=LM_VOCAB, hidden=LM_HIDDEN):
    """Codes + scales of every row, x and the final-norm weights read, logits written."""
    return vocab * (hidden // 2 + (hidden // 32) * 2) + hidden * (4 + 2) + vocab * 4


def run_lm_head(args, ctx):
    """The decode step's lm_head: final RMSNorm + 248,320 Q4 embedding rows
    (tied weights, vocab-major) dotted with one hidden state."""
    K, Wm = args.steps, args.warmup
    vocab, hidden = LM_VOCAB, LM_HIDDEN
    packed = ctx.alloc(vocab * hidden // 2)
    ctx.fill_normal(packed, M.QM_F16, vocab * hidden // 4, 0.0, 1.0, 5001)   # any byte is a code pair
    scales = ctx.alloc(vocab * (hidden // 32) * 2)
    ctx.fill_normal(scales, M.QM_F16, vocab * (hidden // 32), 0.02, 0.004, 5002)
    x = ctx.alloc(hidden * 4)
    ctx.fill_normal(x, M.QM_F32, hidden, 0.0, 1.0, 5003)
    gamma = ctx.alloc(hidden * 2)
    ctx.fill_normal(gamma, M.QM_F16, hidden, 0.0, 0.1, 5004)
    logits = ctx.alloc(vocab * 4)
    tm = Timer(ctx)

    def step():
        ctx.q4_lm_head(vocab, hidden, x, gamma, packed, scales, logits)

    for _ in range(Wm):
        step()
    ctx.sync()
    t0, t1 = ctx.event(), ctx.event()
    wall0 = time.perf_counter()
    t0.record()
    for _ in range(K):
        tm.wrap(step)
    t1.record()
    ctx.sync()
    wall = time.perf_counter() - wall0
    k_ms = tm.mean_ms()
    nbytes = lm_head_bytes()
    return {
        "tokens": K, "total_ms": t0.elapsed_ms(t1), "wall_s": wall,
        "dominant": "qm_q4_lm_head (248320 x 2560, final RMSNorm fused)",
        "roofline": {"bound": "hbm", "achieved": nbytes / (k_ms * 1e-3), "peak": HBM_PEAK,
                     "kernel_ms": k_ms, "bytes_per_launch": nbytes},
        "config": {"workload": "lm_head of one decode token: final RMSNorm + 248320 x 2560 Q4 embedding "
                               "(tied, vocab-major) -> f32 logits",
                   "batch": 1, "seq_len": 1, "global_batch": 1, "parallelism": "single GPU"},
    }


SAMPLE_GEN = 1000
MODEL_POS = 4096          # decode position of the whole-model step
FA_LAYER_PROJ = {"q_proj": (2560, 8192), "k_proj": (2560, 1024), "v_proj": (2560, 1024), "o_proj": (4096, 2560),
                 "gate_proj": (2560, 9216), "up_proj": (2560, 9216), "down_proj": (9216, 2560)}


def _model_on_device(ctx, cap):
    """Random weights of the 4B's real shapes in the device layouts (2.3 GB):
    24 DeltaNet and 8 GQA layers with their Q4 projections, mixer
    parameters, DeltaNet states and f16 KV caches of cap positions, the
    vocab-major Q4 embedding, final norm and RoPE tables."""
    seed = [7000]
    V, H = LM_VOCAB, LM_HIDDEN

    def fill(buf, dtype, count, std, mean=0.0):
        ctx.fill_normal(buf, dtype, count, mean, std, seed[0])
        seed[0] += 1

    def weight(k, n):
        codes = ctx.alloc(k * n // 2)
        fill(codes, M.QM_F16, k * n // 4, 1.0)
        gscales = ctx.alloc(max(16, k * (n // 32) * 2))
        fill(gscales, M.QM_F16, k * (n // 32), 0.0012, 0.006)
        return codes, gscales

    def f16vec(n, mean, std):
        b = ctx.alloc(max(16, n * 2))
        fill(b, M.QM_F16, n, std, mean)
        return b

    rng = np.random.default_rng(8)
    layers = []
    for layer in range(32):
        if layer % 4 != 3:
            p = W.dn_params(rng)
            L = {"dn": True, **{nm: weight(*W.Q4_PROJ_SHAPES[nm]) for nm in Q4_LAYER_PROJ},
                 "conv_w": ctx.upload(p["conv_w"]), "a_log": ctx.upload(p["a_log"]),
                 "dt_bias": ctx.upload(p["dt_bias"]), "attn_norm": ctx.upload(p["norm_w"]),
                 "state": ctx.alloc(32 * 128 * 128 * 4), "conv_buf": ctx.alloc(8192 * 3 * 4)}
            fill(L["state"], M.QM_F32, 32 * 128 * 128, 0.02)
            fill(L["conv_buf"], M.QM_F32, 8192 * 3, 1.0)
        else:
            L = {"dn": False, **{nm: weight(*sh) for nm, sh in FA_LAYER_PROJ.items()},
                 "q_norm": f16vec(256, 0.0, 0.1), "k_norm": f16vec(256, 0.0, 0.1),
                 "kc": ctx.alloc(4 * cap * 256 * 2), "vc": ctx.alloc(4 * cap * 256 * 2)}
            fill(L["kc"], M.QM_F16, 4 * cap * 256, 1.0)
            fill(L["vc"], M.QM_F16, 4 * cap * 256, 1.0)
        L["in_norm"], L["post_norm"] = f16vec(H, 0.0, 0.1), f16vec(H, 0.0, 0.1)
        layers.append(L)
    emb_codes = ctx.alloc(V * H // 2)
    fill(emb_codes, M.QM_F16, V * H // 4, 1.0)
    emb_scales = ctx.alloc(V * (H // 32) * 2)
    fill(emb_scales, M.QM_F16, V * (H // 32), 0.004, 0.02)
    cos, sin = M.rope_table(cap + 1)
    return {"layers": layers, "emb": (emb_codes, emb_scales), "final_norm": f16vec(H, 0.0, 0.1),
            "rope": (ctx.upload(cos), ctx.upload(sin), cap + 1)}


PREFILL_T = 4096


def model_gemm_flops_per_token():
    """2 k n over every projection of the 32 layers (the MLP's gate and up included)."""
    dn = sum(k * n for k, n in (W.Q4_PROJ_SHAPES[nm] for nm in Q4_LAYER_PROJ))
    fa = sum(k * n for k, n in FA_LAYER_PROJ.values())
    return 2 * (24 * dn + 8 * fa)


def run_prefill_model(args, ctx):
    """A 4096-token prompt through the whole 4B model (prefill, gemv.rs:1243-1283):
    embedding rows; per layer RMSNorm to f16, the projections as Q4 GEMMs on
    MFMA (bf16 mixer inputs), the chunked DeltaNet or causal GQA prefill, the
    out/o_proj GEMM on the bf16 mixer output with the residual, RMSNorm, the
    fused gate/up GEMM and the down GEMM with the residual; then the final
    norm and lm_head of the last token.  Random weights of the real shapes."""
    K, Wm = args.steps, args.warmup
    V, H, T = LM_VOCAB, LM_HIDDEN, PREFILL_T
    mdl = _model_on_device(ctx, T)
    layers, (emb_codes, emb_scales), final_norm = mdl["layers"], mdl["emb"], mdl["final_norm"]
    rc, rs, rope_len = mdl["rope"]
    ids = ctx.upload(np.random.default_rng(9).integers(0, V, T).astype(np.int32))
    x, xn = ctx.alloc(T * H * 4), ctx.alloc(T * H * 2)
    proj, z16, mix16 = ctx.alloc(T * 8192 * 2), ctx.alloc(T * 4096 * 2), ctx.alloc(T * 4096 * 2)
    a, b, k16, v16 = ctx.alloc(T * 32 * 4), ctx.alloc(T * 32 * 4), ctx.alloc(T * 1024 * 2), ctx.alloc(T * 1024 * 2)
    inter_bf16, logits = ctx.alloc(T * 9216 * 2), ctx.alloc(V * 4)
    ctx.reserve(max_batch=1, max_kv_len=T, max_prefill_tokens=T)
    ctx.sync()
    gemm_timer = Timer(ctx)

    def step():
        ctx.q4_embed(T, V, H, ids, emb_codes, emb_scales, x)
        for L in layers:
            ctx.rms_norm_f16(T, H, x, L["in_norm"], xn)
            if L["dn"]:
                ctx.q4_gemm(T, H, 8192, xn, *L["in_proj_qkv"], y_bf16=proj)
                ctx.q4_gemm(T, H, 4096, xn, *L["in_proj_z"], y_bf16=z16)
                ctx.q4_gemm(T, H, 32, xn, *L["in_proj_a"], y=a)
                ctx.q4_gemm(T, H, 32, xn, *L["in_proj_b"], y=b)
                ctx.deltanet_prefill(T, proj, L["conv_buf"], L["conv_w"], a, b, L["a_log"], L["dt_bias"], z16,
                                     L["attn_norm"], L["state"], mix16)
                ctx.q4_gemm(T, 4096, H, mix16, *L["out_proj"], y=x, residual=x, x_dtype=M.QM_BF16)
            else:
                ctx.q4_gemm(T, H, 8192, xn, *L["q_proj"], y_bf16=proj)
                ctx.q4_gemm(T, H, 1024, xn, *L["k_proj"], y_bf16=k16)
                ctx.q4_gemm(T, H, 1024, xn, *L["v_proj"], y_bf16=v16)
                ctx.gqa_prefill(T, proj, k16, v16, L["q_norm"], L["k_norm"], rc, rs, rope_len, L["kc"], L["vc"], T,
                                mix16)
                ctx.q4_gemm(T, 4096, H, mix16, *L["o_proj"], y=x, residual=x, x_dtype=M.QM_BF16)
            ctx.rms_norm_f16(T, H, x, L["post_norm"], xn)
            ctx.q4_gemm_gate_up(T, H, 9216, xn, *L["gate_proj"], *L["up_proj"], inter_bf16)
            ctx.q4_gemm(T, 9216, H, inter_bf16, *L["down_proj"], y=x, residual=x, x_dtype=M.QM_BF16)
        ctx.q4_lm_head(V, H, x.offset((T - 1) * H * 4), final_norm, emb_codes, emb_scales, logits)

    for _ in range(Wm):
        step()
    ctx.sync()
    t0, t1 = ctx.event(), ctx.event()
    wall0 = time.perf_counter()
    t0.record()
    for _ in range(K):
        step()
    t1.record()
    ctx.sync()
    wall = time.perf_counter() - wall0
    ms = t0.elapsed_ms(t1) / K
    flops = model_gemm_flops_per_token() * T
    return {
        "tokens": K * T, "total_ms": t0.elapsed_ms(t1), "wall_s": wall,
        "dominant": "whole prefill (embedding, 32 layers of Q4 GEMMs + chunked mixers, lm_head)",
        "roofline": {"bound": "mfma", "achieved": flops / (ms * 1e-3), "peak": MFMA_BF16_PEAK,
                     "kernel_ms": ms, "flops_per_launch": flops},
        "config": {"workload": "whole-model prefill of a 4096-token prompt: embedding, 24 DeltaNet + 8 GQA layers "
                               "(Q4 projection GEMMs on MFMA with f16/bf16 activations, chunked DeltaNet and causal "
                               "GQA prefill), lm_head of the last token; roofline over the projection GEMM flops",
                   "batch": 1, "seq_len": T, "global_batch": 1, "parallelism": "single GPU"},
    }


def run_decode_model(args, ctx):
    """One decode token through the whole 4B model at batch 1, position 4096:
    embedding row, 24 DeltaNet and 8 GQA layers (input RMSNorm + projections,
    mixer, out/o_proj residual, RMSNorm + gate/up MLP, down residual), final
    RMSNorm + lm_head over 248,320 rows, and top-k sampling whose token feeds
    the next step's embedding on the device (forward_decode, gemv.rs:1059-1077,
    then sample_token_top_k).  Random weights of the real shapes (2.3 GB
    resident), captured once as a HIP graph and replayed."""
    K, Wm = args.steps, args.warmup
    V, H, P = LM_VOCAB, LM_HIDDEN, MODEL_POS
    cap = P + 1
    mdl = _model_on_device(ctx, cap)
    layers, (emb_codes, emb_scales), final_norm = mdl["layers"], mdl["emb"], mdl["final_norm"]
    rc, rs, _ = mdl["rope"]
    tok = ctx.upload(np.array([1234, 0, 0, 0], np.int32))
    rng_state = ctx.upload(np.array([0x9E3779B97F4A7C15], np.uint64))
    x, proj, z = ctx.alloc(H * 4), ctx.alloc(8192 * 4), ctx.alloc(4096 * 4)
    a, b, kn, vn = ctx.alloc(32 * 4), ctx.alloc(32 * 4), ctx.alloc(1024 * 4), ctx.alloc(1024 * 4)
    mix, inter, logits = ctx.alloc(4096 * 4), ctx.alloc(9216 * 4), ctx.alloc(V * 4)
    ctx.reserve(max_batch=1, max_kv_len=cap)
    ctx.sync()

    def step():
        ctx.q4_embed(1, V, H, tok, emb_codes, emb_scales, x)
        for L in layers:
            if L["dn"]:
                # the conv1d step + SiLU ride on the in_proj_qkv launch
                ctx.q4_gemv_multi(H, x, [(8192, *L["in_proj_qkv"], proj), (4096, *L["in_proj_z"], z),
                                         (32, *L["in_proj_a"], a), (32, *L["in_proj_b"], b)], norm_w=L["in_norm"],
                                  conv_buf=L["conv_buf"], conv_w=L["conv_w"])
                ctx.deltanet_decode(1, M.QM_DN_POSTACT, proj, None, None, a, b, L["a_log"],
                                    L["dt_bias"], z, L["attn_norm"], L["state"], mix)
                ctx.q4_gemv_multi(4096, mix, [(H, *L["out_proj"], x, x)])
            else:
                ctx.q4_gemv_multi(H, x, [(8192, *L["q_proj"], proj), (1024, *L["k_proj"], kn),
                                         (1024, *L["v_proj"], vn)], norm_w=L["in_norm"])
                ctx.gqa_decode(1, proj, kn, vn, L["q_norm"], L["k_norm"], rc, rs, cap + 1, None, P,
                               L["kc"], L["vc"], cap, mix)
                ctx.q4_gemv_multi(4096, mix, [(H, *L["o_proj"], x, x)])
            ctx.q4_gate_up(H, 9216, x, L["post_norm"], *L["gate_proj"], *L["up_proj"], inter)
            ctx.q4_gemv_multi(9216, inter, [(H, *L["down_proj"], x, x)])
        ctx.q4_lm_head(V, H, x, final_norm, emb_codes, emb_scales, logits)
        ctx.sample(V, logits, None, 0, rng_state, tok, temperature=1.0, top_p=0.95, top_k=20)

    for _ in range(Wm):
        step()
    ctx.sync()
    t0, t1 = ctx.event(), ctx.event()
    wall0 = time.perf_counter()
    t0.record()
    for _ in range(K):
        step()
    t1.record()
    ctx.sync()
    eager_ms = t0.elapsed_ms(t1) / K
    total_ms, wall = t0.elapsed_ms(t1), time.perf_counter() - wall0
    graph_ms = float("nan")
    if not args.no_graph:
        ctx.graph_begin()
        step()
        g = ctx.graph_end()
        g.launch()
        ctx.sync()
        g0, g1 = ctx.event(), ctx.event()
        wall0 = time.perf_counter()
        g0.record()
        for _ in range(K):
            g.launch()
        g1.record()
        ctx.sync()
        wall = time.perf_counter() - wall0
        total_ms = g0.elapsed_ms(g1)
        graph_ms = total_ms / K
    wbytes = (24 * sum(q4_weight_bytes(*W.Q4_PROJ_SHAPES[nm]) for nm in Q4_LAYER_PROJ)
              + 8 * sum(q4_weight_bytes(*sh) for sh in FA_LAYER_PROJ.values()))
    nbytes = (wbytes + lm_head_bytes() + 24 * 2 * 32 * 128 * 128 * 4    # weights, lm_head, state read + write
              + 8 * 2 * 4 * cap * 256 * 2)                              # K and V read
    ms = total_ms / K
    return {
        "tokens": K, "total_ms": total_ms, "wall_s": wall,
        "dominant": "whole decode step (embedding, 32 layers, lm_head, sampling)" +
                    (" as one HIP graph" if not args.no_graph else ", eager"),
        "roofline": {"bound": "hbm", "achieved": nbytes / (ms * 1e-3), "peak": HBM_PEAK,
                     "kernel_ms": ms, "bytes_per_launch": nbytes},
        "eager_ms_per_step": eager_ms, "graph_ms_per_step": graph_ms,
        "config": {"workload": "whole-model decode, batch 1, position 4096: embedding, 24 DeltaNet + 8 GQA layers "
                               "with Q4 projections and MLPs, final RMSNorm + lm_head (248320 x 2560), top-k 20 "
                               "sampling feeding the next token on the device",
                   "batch": 1, "seq_len": P, "global_batch": 1, "parallelism": "single GPU"},
    }


def run_sample(args, ctx):
    """Next-token sampling over the 248,320 logits of one decode step with
    the reference's defaults (temperature 1, top_p 0.95, top_k 20, presence
    penalty 1.5 over 1000 generated ids), logits resident in HBM."""
    K, Wm = args.steps, args.warmup
    V = LM_VOCAB
    logits = ctx.alloc(V * 4)
    ctx.fill_normal(logits, M.QM_F32, V, 0.0, 3.0, 6001)
    gen = ctx.upload(np.random.default_rng(6002).integers(0, V, SAMPLE_GEN).astype(np.int32))
    state = ctx.upload(np.array([0x9E3779B97F4A7C15], np.uint64))
    tok = ctx.alloc(4)
    ctx.reserve(1, 0, 0)

    def step():
        ctx.sample(V, logits, gen, SAMPLE_GEN, state, tok, temperature=1.0, top_p=0.95, top_k=20,
                   presence_penalty=1.5)

    for _ in range(Wm):
        step()
    ctx.sync()
    t0, t1 = ctx.event(), ctx.event()
    wall0 = time.perf_counter()
    t0.record()
    for _ in range(K):
        step()
    t1.record()
    ctx.sync()
    wall = time.perf_counter() - wall0
    ms = t0.elapsed_ms(t1) / K
    nbytes = V * 4 * 2 + SAMPLE_GEN * 4       # logits read by the penalty pass and the selection
    return {
        "tokens": K, "total_ms": t0.elapsed_ms(t1), "wall_s": wall,
        "dominant": "qm_sample (penalties + select + merge/draw, 3 launches)",
        "roofline": {"bound": "hbm", "achieved": nbytes / (ms * 1e-3), "peak": HBM_PEAK,
                     "kernel_ms": ms, "bytes_per_launch": nbytes},
        "config": {"workload": "next-token sampling over 248320 logits: presence penalty (1000 ids), top_k 20, "
                               "top_p 0.95, temperature 1",
                   "batch": 1, "seq_len": 1, "global_batch": 1, "parallelism": "single GPU"},
    }


def _repeat_for(fn, min_s=None, max_iters=10 ** 6):
    """Call fn() until min_s (default CPU_SAMPLE_S) seconds have elapsed;
    returns (calls, seconds)."""
    min_s = CPU_SAMPLE_S if min_s is None else min_s
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= min_s or n >= max_iters:
            return n, dt


def host_cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(workload: str) -> dict:
    """The oracle on this host's cores, plus what the reference prints about
    the host (simd.rs:18-27): the CPU model and its AVX-512 detection."""
    O = _load("qora_oracle_py", ROOT / "oracle" / "oracle.py")
    r = _cpu_baseline(workload, O)
    r["cpu_model"] = host_cpu_model()
    r["avx512"] = bool(O.has_avx512())
    r["host_cores"] = host_cores()
    return r


def _cpu_baseline(workload: str, O) -> dict:
    cores = host_cores()
    att_threads = min(16, cores)
    cfg = O.config()
    avx = "AVX-512" if O.has_avx512() else "scalar"
    if workload == "dn_decode":
        steps = 256
        w = W.dn_decode_workload(steps, 1, seed=0)
        S = w["state0"][0].copy()

        def sample():
            for t in range(steps):
                O.deltanet_decode_step(cfg, w["qkv"][t, 0], w["a"][t, 0], w["b"][t, 0], w["z"][t, 0],
                                       w["conv_w"], w["a_log"], w["dt_bias"], w["norm_w"], S)
        n, dt = _repeat_for(sample)
        res = {"value": n * steps / dt, "unit": "tokens/s", "cores": 1, "kind": "port",
               "sample": f"{n} x 256 decode steps, batch 1, {avx} head update, 1 thread ({dt:.1f} s)"}
        # a stronger CPU figure than the reference's serial head loop
        # (gemv.rs:817): the 32 v-heads of each step over all host cores
        S2 = w["state0"][0].copy()

        def sample_mt():
            for t in range(steps):
                O.deltanet_decode_step(cfg, w["qkv"][t, 0], w["a"][t, 0], w["b"][t, 0], w["z"][t, 0],
                                       w["conv_w"], w["a_log"], w["dt_bias"], w["norm_w"], S2,
                                       nthreads=att_threads)
        n2, dt2 = _repeat_for(sample_mt, min_s=max(CPU_SAMPLE_S / 2, 2.0))
        res["all_cores_heads_parallel"] = {
            "value": n2 * steps / dt2, "unit": "tokens/s", "cores": att_threads,
            "label": "stronger than the reference: its v-head loop (gemv.rs:817) is serial",
            "sample": f"{n2} x 256 decode steps, v-heads over {att_threads} threads (the host's "
                      f"CPU share for one GPU), {avx} head update ({dt2:.1f} s)"}
        return res
    if workload == "dn_prefill":
        T = 1024
        w = W.dn_prefill_workload(T, seed=2)
        S, buf = w["state0"].copy(), w["conv_buf0"].copy()
        qkv, z = W.bf16_value(w["qkv"]), W.bf16_value(w["z"])

        def sample():
            O.deltanet_prefill(cfg, qkv, w["a"], w["b"], z, w["conv_w"], w["a_log"], w["dt_bias"],
                               w["norm_w"], S, buf)
        n, dt = _repeat_for(sample)
        return {"value": n * T / dt, "unit": "tokens/s", "cores": 1, "kind": "port",
                "sample": f"{n} x sequential prefill of 1024 tokens (gemv.rs:1119-1219 scalar loop, "
                          f"1 thread; per-token cost is independent of position) ({dt:.1f} s)"}
    if workload == "gqa_prefill":
        S = 8192
        w = W.gqa_prefill_workload(S, seed=3)
        cos, sin = O.rope_table(S)
        qg = W.bf16_value(w["q_gate"]).reshape(S, -1)
        kk = W.bf16_value(w["k"]).reshape(S, -1)
        vv = W.bf16_value(w["v"]).reshape(S, -1)
        done = {"rows": 0.0, "pairs": 0.0}

        def sample():
            hi = S - 16 * int(done["rows"] // 16)
            rows = np.arange(max(hi - 16, 0), hi)
            O.attn_prefill(cfg, qg, kk, vv, w["q_norm"], w["k_norm"], cos, sin, rows=rows,
                           nthreads=att_threads)
            done["rows"] += len(rows)
            done["pairs"] += float(np.sum(rows + 1))
        n, dt = _repeat_for(sample, max_iters=S // 16)
        full = S * (S + 1) / 2.0
        return {"value": S / (dt * full / done["pairs"]), "unit": "tokens/s", "cores": att_threads,
                "kind": "port",
                "sample": f"{int(done['rows'])} of the last rows of the 8192-token causal prefill "
                          f"(gemv.rs:1402-1444), heads over {att_threads} threads, extrapolated "
                          f"linearly in row-key pairs ({dt:.1f} s)"}
    if workload == "q4_proj":
        rng = np.random.default_rng(8)
        ws = {nm: W.q4_random_weight(*W.Q4_PROJ_SHAPES[nm], rng) for nm in Q4_LAYER_PROJ}
        x = rng.standard_normal(2560, dtype=np.float32)
        mix = rng.standard_normal(4096, dtype=np.float32)
        gam = W.f16_bits(0.1 * rng.standard_normal(2560, dtype=np.float32))

        def sample():
            xn = O.rms_norm(x, gam)
            for nm in ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b"):
                O.q4_gemv(xn, *ws[nm])
            h = x + O.q4_gemv(mix, *ws["out_proj"])
            inter = O.q4_gate_up(O.rms_norm(h, gam), *ws["gate_proj"], *ws["up_proj"])
            O.q4_gemv(inter, *ws["down_proj"])
        n, dt = _repeat_for(sample)
        return {"value": n / dt / Q4_LAYERS, "unit": "tokens/s", "cores": 1, "kind": "port",
                "sample": f"{n} DeltaNet-layer sets of the Q4 projections, norms and residuals "
                          f"(scalar gemv_q4_inner restatement, one thread, {dt:.1f} s); "
                          f"tokens/s = layer sets/s / 24"}
    if workload == "q4_gemm":
        rng = np.random.default_rng(9)
        packed, scales = W.q4_random_weight(*W.Q4_PROJ_SHAPES["in_proj_qkv"], rng)
        xs = W.f16_value(W.f16_bits(rng.standard_normal((8, 2560), dtype=np.float32)))
        n, dt = _repeat_for(lambda: O.q4_gemm(xs, packed, scales, nthreads=1))
        return {"value": 8 * n / dt, "unit": "tokens/s", "cores": 1, "kind": "port",
                "sample": f"{n} calls of gemm_q4 on 8 rows (scalar gemv_q4_inner restatement, one thread, "
                          f"{dt:.1f} s)"}
    if workload == "decode_model":
        # one DeltaNet and one GQA layer (projections, mixer, MLP) and the
        # lm_head, timed separately; tokens/s = 1 / (24 t_dn + 8 t_gqa + t_head)
        rng = np.random.default_rng(12)
        dw = {nm: W.q4_random_weight(*W.Q4_PROJ_SHAPES[nm], rng) for nm in Q4_LAYER_PROJ}
        fw = {nm: W.q4_random_weight(*sh, rng) for nm, sh in FA_LAYER_PROJ.items()}
        p = W.dn_params(rng)
        gam = W.f16_bits(0.1 * rng.standard_normal(2560, dtype=np.float32))
        qn = W.f16_bits(0.1 * rng.standard_normal(256, dtype=np.float32))
        x = rng.standard_normal(2560, dtype=np.float32)
        S = 0.02 * rng.standard_normal((32, 128, 128), dtype=np.float32)
        cbuf = rng.standard_normal((8192, 3), dtype=np.float32)
        cos, sin = O.rope_table(MODEL_POS + 1)
        Kc = W.f16_value(W.f16_bits(rng.standard_normal((MODEL_POS + 1, 4, 256), dtype=np.float32)))
        Vc = W.f16_value(W.f16_bits(rng.standard_normal((MODEL_POS + 1, 4, 256), dtype=np.float32)))

        def mlp(h):
            inter = O.q4_gate_up(O.rms_norm(h, gam), *dw["gate_proj"], *dw["up_proj"])
            return h + O.q4_gemv(inter, *dw["down_proj"])

        def dn_layer():
            xn = O.rms_norm(x, gam)
            qkv, z = O.q4_gemv(xn, *dw["in_proj_qkv"]), O.q4_gemv(xn, *dw["in_proj_z"])
            av, bv = O.q4_gemv(xn, *dw["in_proj_a"]), O.q4_gemv(xn, *dw["in_proj_b"])
            out = O.deltanet_decode_step(cfg, qkv, av, bv, z, p["conv_w"], p["a_log"], p["dt_bias"], p["norm_w"],
                                         S, conv_buf=cbuf, preact=True)
            return mlp(x + O.q4_gemv(out, *dw["out_proj"]))

        def gqa_layer():
            xn = O.rms_norm(x, gam)
            qg, kk, vv = (O.q4_gemv(xn, *fw[nm]) for nm in ("q_proj", "k_proj", "v_proj"))
            out = O.attn_decode_step(cfg, qg, kk, vv, qn, qn, cos, sin, Kc, Vc, MODEL_POS, nthreads=att_threads)
            return mlp(x + O.q4_gemv(out, *fw["o_proj"]))

        ep, es = W.q4_random_weight(LM_VOCAB, LM_HIDDEN, rng, scale=0.02)
        n1, t_dn = _repeat_for(dn_layer, min_s=4.0)
        n2, t_fa = _repeat_for(gqa_layer, min_s=4.0)
        n3, t_hd = _repeat_for(lambda: O.q4_lm_head(O.rms_norm(x, gam), ep, es, nthreads=att_threads), min_s=2.0)
        per_token = 24 * t_dn / n1 + 8 * t_fa / n2 + t_hd / n3
        return {"value": 1.0 / per_token, "unit": "tokens/s", "cores": att_threads, "kind": "port",
                "sample": f"{n1} DeltaNet layers, {n2} GQA layers (position 4096, heads over {att_threads} "
                          f"threads) and {n3} lm_heads timed separately (projections by the scalar gemv_q4_inner "
                          f"restatement, one thread); tokens/s = 1 / (24 t_dn + 8 t_gqa + t_head); "
                          f"{per_token:.2f} s per token"}
    if workload == "prefill_model":
        # one DeltaNet and one GQA layer prefilled over an 8-token prompt
        # (gemm_q4 = 8 row gemvs, the sequential DeltaNet prefill, causal
        # attention), scaled linearly to 24 + 8 layers
        rng = np.random.default_rng(13)
        Tc = 8
        dw = {nm: W.q4_random_weight(*W.Q4_PROJ_SHAPES[nm], rng) for nm in Q4_LAYER_PROJ}
        fw = {nm: W.q4_random_weight(*sh, rng) for nm, sh in FA_LAYER_PROJ.items()}
        p = W.dn_params(rng)
        gam = W.f16_bits(0.1 * rng.standard_normal(2560, dtype=np.float32))
        qn = W.f16_bits(0.1 * rng.standard_normal(256, dtype=np.float32))
        X = rng.standard_normal((Tc, 2560), dtype=np.float32)
        cos, sin = O.rope_table(Tc + 1)

        def rows(f, A):
            return np.stack([f(r) for r in A])

        def mlp(h, ws):
            hn = rows(lambda r: O.rms_norm(r, gam), h)
            g, u = O.q4_gemm(hn, *ws["gate_proj"], nthreads=1), O.q4_gemm(hn, *ws["up_proj"], nthreads=1)
            return h + O.q4_gemm((g / (1.0 + np.exp(-g)) * u).astype(np.float32), *ws["down_proj"], nthreads=1)

        def dn_layer():
            xn = rows(lambda r: O.rms_norm(r, gam), X)
            qkv, z = O.q4_gemm(xn, *dw["in_proj_qkv"], nthreads=1), O.q4_gemm(xn, *dw["in_proj_z"], nthreads=1)
            av, bv = O.q4_gemm(xn, *dw["in_proj_a"], nthreads=1), O.q4_gemm(xn, *dw["in_proj_b"], nthreads=1)
            out = O.deltanet_prefill(cfg, qkv, av, bv, z, p["conv_w"], p["a_log"], p["dt_bias"], p["norm_w"],
                                     np.zeros((32, 128, 128), np.float32), np.zeros((8192, 3), np.float32))
            return mlp(X + O.q4_gemm(out, *dw["out_proj"], nthreads=1), dw)

        def gqa_layer():
            xn = rows(lambda r: O.rms_norm(r, gam), X)
            qg, kk, vv = (O.q4_gemm(xn, *fw[nm], nthreads=1) for nm in ("q_proj", "k_proj", "v_proj"))
            out = O.attn_prefill(cfg, qg, kk, vv, qn, qn, cos, sin, nthreads=att_threads)[0]
            return mlp(X + O.q4_gemm(out, *fw["o_proj"], nthreads=1), fw)

        n1, t_dn = _repeat_for(dn_layer, min_s=4.0)
        n2, t_fa = _repeat_for(gqa_layer, min_s=4.0)
        per_prompt = 24 * t_dn / n1 + 8 * t_fa / n2
        return {"value": Tc / per_prompt, "unit": "tokens/s", "cores": 1, "kind": "port",
                "sample": f"{n1} DeltaNet and {n2} GQA layer prefills of an {Tc}-token prompt timed separately "
                          f"(gemm_q4 as row gemvs, the sequential DeltaNet prefill, one thread), scaled to "
                          f"24 + 8 layers: tokens/s = {Tc} / (24 t_dn + 8 t_gqa)"}
    if workload == "sample":
        rng = np.random.default_rng(11)
        x = (3.0 * rng.standard_normal(LM_VOCAB)).astype(np.float32)
        gen = rng.integers(0, LM_VOCAB, SAMPLE_GEN).astype(np.int32)
        st = np.array([12345], np.uint64)
        n, dt = _repeat_for(lambda: O.sample_top_k(O.apply_penalties(x, gen, 1.0, 1.5), 1.0, 0.95, 20, st))
        return {"value": n / dt, "unit": "tokens/s", "cores": 1, "kind": "port",
                "sample": f"{n} samplings (presence penalty, full stable sort of 248320 logits, softmax, top-p, "
                          f"draw; generate.rs restatement, one thread, {dt:.1f} s)"}
    if workload == "lm_head":
        rng = np.random.default_rng(10)
        packed, scales = W.q4_random_weight(LM_VOCAB, LM_HIDDEN, rng, scale=0.02)
        x = rng.standard_normal(LM_HIDDEN, dtype=np.float32)
        gam = W.f16_bits(0.1 * rng.standard_normal(LM_HIDDEN, dtype=np.float32))
        n, dt = _repeat_for(lambda: O.q4_lm_head(O.rms_norm(x, gam), packed, scales, nthreads=att_threads))
        return {"value": n / dt, "unit": "tokens/s", "cores": att_threads, "kind": "port",
                "sample": f"{n} full lm_heads (rms_norm + 248320 x 2560 Q4 rows, lm_head_parallel restatement, "
                          f"rows over {att_threads} threads, {dt:.1f} s)"}
    if workload == "gqa_decode":
        pos = 4096
        w = W.gqa_decode_workload(pos, 1, seed=1)
        cos, sin = O.rope_table(pos + 1)
        K = np.ascontiguousarray(np.transpose(W.f16_value(w["k_cache"][0]), (1, 0, 2)))
        V = np.ascontiguousarray(np.transpose(W.f16_value(w["v_cache"][0]), (1, 0, 2)))

        def sample():
            O.attn_decode_step(cfg, w["q_gate"][0].ravel(), w["k_new"][0].ravel(), w["v_new"][0].ravel(),
                               w["q_norm"], w["k_norm"], cos, sin, K, V, pos, nthreads=att_threads)
        n, dt = _repeat_for(sample)
        return {"value": n / dt, "unit": "tokens/s", "cores": att_threads, "kind": "port",
                "sample": f"{n} decode steps at position 4096, f32 KV, heads over {att_threads} threads ({dt:.1f} s)"}
    # stack: one sequence decoding through all 32 layers at context 32768
    max_steps, ctx0 = 64, 32768
    rng = np.random.default_rng(7)
    cos, sin = O.rope_table(ctx0 + max_steps + 1)
    dn_w = [W.dn_params(rng) for _ in range(N_DN)]
    dn_S = [(0.02 * rng.standard_normal((32, 128, 128), dtype=np.float32)) for _ in range(N_DN)]
    caches = []
    for _ in range(N_GQA):
        Kc = np.empty((ctx0 + max_steps, 4, 256), np.float32)
        Vc = np.empty_like(Kc)
        Kc[:ctx0] = W.f16_value(W.f16_bits(rng.standard_normal((ctx0, 4, 256), dtype=np.float32)))
        Vc[:ctx0] = W.f16_value(W.f16_bits(rng.standard_normal((ctx0, 4, 256), dtype=np.float32)))
        caches.append((Kc, Vc))
    qn = W.f16_bits(0.1 * rng.standard_normal(256, dtype=np.float32))
    dn_in = rng.standard_normal((max_steps, N_DN, 8192 + 32 + 32 + 4096), dtype=np.float32)
    g_in = rng.standard_normal((max_steps, N_GQA, 16 * 512 + 2 * 1024), dtype=np.float32)
    state = {"s": 0}

    def sample():
        s = state["s"]
        li_dn = li_g = 0
        for layer in range(32):
            if layer % 4 != 3:
                p, x = dn_w[li_dn], dn_in[s, li_dn]
                O.deltanet_decode_step(cfg, x[:8192], x[8192:8224], x[8224:8256], x[8256:],
                                       p["conv_w"], p["a_log"], p["dt_bias"], p["norm_w"], dn_S[li_dn])
                li_dn += 1
            else:
                Kc, Vc = caches[li_g]
                x = g_in[s, li_g]
                O.attn_decode_step(cfg, x[:8192], x[8192:9216], x[9216:], qn, qn, cos, sin,
                                   Kc, Vc, ctx0 + s, nthreads=att_threads)
                li_g += 1
        state["s"] += 1
    n, dt = _repeat_for(sample, max_iters=max_steps)
    return {"value": n / dt, "unit": "tokens/s", "cores": att_threads, "kind": "port",
            "sample": f"1 sequence x {n} decode steps through 32 layers at context {ctx0}; "
                      f"f32 KV (the reference's storage), attention heads over {att_threads} threads, "
                      f"DeltaNet heads serial ({avx} update) ({dt:.1f} s)"}


# The per-config sub-results of the default line: each single-layer workload
# of the metric at its own default step counts, with its CPU baseline on a
# shorter sample than the headline's.
SUB_CONFIGS = (("dn_decode_b1", "dn_decode"), ("gqa_decode_b1_pos4096", "gqa_decode"),
               ("dn_prefill_seq4096", "dn_prefill"), ("gqa_prefill_seq8192", "gqa_prefill"))
SUB_CPU_SAMPLE_S = 5.0
DEFAULT_STEPS = {"stack": (32, 4), "dn_decode": (256, 16), "gqa_decode": (200, 20),
                 "dn_prefill": (20, 3), "gqa_prefill": (10, 2), "q4_proj": (50, 5), "q4_gemm": (20, 3),
                 "lm_head": (100, 10), "sample": (200, 10), "decode_model": (30, 3),
                 "prefill_model": (5, 1)}
RUNNERS = {"stack": "run_stack", "dn_decode": "run_dn_decode", "gqa_decode": "run_gqa_decode",
           "dn_prefill": "run_dn_prefill", "gqa_prefill": "run_gqa_prefill", "q4_proj": "run_q4_proj",
           "q4_gemm": "run_q4_gemm", "lm_head": "run_lm_head", "sample": "run_sample",
           "decode_model": "run_decode_model", "prefill_model": "run_prefill_model"}


def roofline_of(r: dict) -> dict:
    roof = r["roofline"]
    if roof["bound"] == "mfma":
        return {"bound": "mfma", "achieved": roof["achieved"] / 1e12, "peak": roof["peak"] / 1e12,
                "unit": "TFLOP/s", "frac": roof["achieved"] / roof["peak"], "traffic": None,
                "kernel": r["dominant"], "kernel_avg_ms": roof["kernel_ms"],
                "flops_per_launch": roof["flops_per_launch"]}
    return {"bound": roof["bound"], "achieved": roof["achieved"] / 1e9, "peak": roof["peak"] / 1e9,
            "unit": "GB/s", "frac": roof["achieved"] / roof["peak"], "traffic": None,
            "kernel": r["dominant"], "kernel_avg_ms": roof["kernel_ms"],
            "bytes_per_launch": roof["bytes_per_launch"]}


def code_hash(sources):
    """sha256 over the sources with comments and blank space removed (so a
    comment edit does not invalidate a measurement of the code)."""
    import hashlib
    import re
    h = hashlib.sha256()
    for src in sources:
        text = (ROOT / src).read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        h.update(re.sub(r"\s+", " ", text).strip().encode())
    return h


def stored_traffic(kernel_sources) -> dict:
    """HBM bytes per launch of the stack's GQA decode from the committed
    rocprofv3 --pmc calibration, used only while the kernel sources it was
    measured on are unchanged (their sha256 is stored beside the figure)."""
    tf = ROOT / "profiles" / "traffic_stack_gqa_decode.json"
    if not tf.exists():
        return {"traffic": None, "traffic_source": "no stored rocprofv3 calibration"}
    rec = json.loads(tf.read_text())
    h = code_hash(kernel_sources)
    if rec.get("sources_sha256") != h.hexdigest():
        return {"traffic": None,
                "traffic_source": "stored rocprofv3 calibration is stale (kernel sources changed since)"}
    return {"traffic": rec["traffic_bytes_per_launch"],
            "traffic_source": "stored: rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE of this workload, scaled by a "
                              "1 GiB copy (profiles/traffic_stack_gqa_decode.json), valid for the unchanged "
                              "kernel sources (sha256 " + h.hexdigest()[:16] + ")"}


def sub_config(name: str, workload: str, ctx, with_cpu: bool) -> dict:
    ns = argparse.Namespace(steps=DEFAULT_STEPS[workload][0], warmup=DEFAULT_STEPS[workload][1],
                            no_graph=False)
    r = globals()[RUNNERS[workload]](ns, ctx)
    ctx.sync()
    rl = roofline_of(r)
    out = {"workload": r["config"]["workload"], "steps": ns.steps, "warmup": ns.warmup,
           "ms": rl["kernel_avg_ms"], "tokens_per_s": r["tokens"] / (r["total_ms"] * 1e-3),
           "roofline": {k: rl[k] for k in ("bound", "achieved", "peak", "unit", "frac", "kernel")}}
    if "eager_event_ms_per_launch" in r:
        # the per-launch variant: HIP events around single eager launches
        # (at batch 1 this includes the host's submission gap between launches)
        out["eager_ms_per_launch"] = r["eager_event_ms_per_launch"]
        out["ms_note"] = "ms: graph-replayed steps (warm, working set in L2 / MALL)"
    if "cold" in r:
        out["cold"] = r["cold"]
    if with_cpu:
        global CPU_SAMPLE_S
        saved, CPU_SAMPLE_S = CPU_SAMPLE_S, SUB_CPU_SAMPLE_S
        try:
            out["cpu_baseline"] = cpu_baseline(workload)
        finally:
            CPU_SAMPLE_S = saved
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="stack",
                    choices=["stack", "dn_decode", "gqa_decode", "dn_prefill", "gqa_prefill", "q4_proj",
                             "q4_gemm", "lm_head", "sample", "decode_model", "prefill_model"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-sub-configs", action="store_true",
                    help="stack only: skip the single-layer sub-results (DeltaNet / GQA decode at batch 1, "
                         "DeltaNet prefill of 4096 tokens, GQA prefill of 8192 tokens)")
    ap.add_argument("--no-graph", action="store_true",
                    help="skip the graph-replayed timing, e.g. to profile the q4_proj workload from eager "
                         "launches (a traced replay of its captured step once ended in a host-side SIGSEGV "
                         "inside the tracer's hipGraphLaunch callback)")
    ap.add_argument("--gqa-chunk", type=int, default=0,
                    help="keys per GQA decode split workgroup (multiple of 64; 0 = the library's choice)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="before timing, copy 1 GiB device-to-device once (a dispatch of known "
                         "traffic for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--code-hash", action="store_true",
                    help="print the comment-insensitive sha256 of the GQA decode sources (stored beside a "
                         "traffic measurement) and exit")
    args = ap.parse_args()
    if args.code_hash:
        print(code_hash(GQA_DECODE_SOURCES).hexdigest())
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: the mixer path here is a single-GPU build "
              "(sharding is a design note, not a launched path); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    defaults = DEFAULT_STEPS[args.workload]
    args.steps = args.steps or defaults[0]
    args.warmup = defaults[1] if args.warmup is None else args.warmup

    ctx = M.Context(0)
    if args.gqa_chunk:
        ctx.set_option(M.QM_OPT_GQA_DECODE_CHUNK, args.gqa_chunk)
    if args.calibrate_copy:
        src, dst = ctx.alloc(1 << 30), ctx.alloc(1 << 30)
        ctx.fill_normal(src, M.QM_F32, (1 << 30) // 4, 0.0, 1.0, 7)
        ctx.copy(dst, src, 1 << 30)
        ctx.sync()
        src.close()
        dst.close()
    r = globals()[RUNNERS[args.workload]](args, ctx)
    ctx.sync()
    subs = None
    if args.workload == "stack" and not args.no_sub_configs:
        import gc
        gc.collect()                      # the stack's 72 GB of buffers
        subs = {}
        for name, wl in SUB_CONFIGS:
            subs[name] = sub_config(name, wl, ctx, with_cpu=not args.no_cpu_baseline)
            gc.collect()
    ctx.close()

    value = r["tokens"] / (r["total_ms"] * 1e-3)
    rl = roofline_of(r)
    line = {
        "metric": {"stack": "mixer tokens/s (decode, 32-layer hybrid stack) on 1x MI355X",
                   "dn_prefill": "mixer tokens/s (prefill) on 1x MI355X",
                   "gqa_prefill": "mixer tokens/s (prefill) on 1x MI355X",
                   "q4_proj": "Q4 projection tokens/s (decode) on 1x MI355X",
                   "q4_gemm": "Q4 projection tokens/s (prefill) on 1x MI355X",
                   "lm_head": "lm_head tokens/s (decode) on 1x MI355X",
                   "sample": "sampled tokens/s (decode) on 1x MI355X",
                   "decode_model": "whole-model decode tokens/s (batch 1) on 1x MI355X",
                   "prefill_model": "whole-model prefill tokens/s on 1x MI355X"}.get(
                       args.workload, "mixer tokens/s (decode) on 1x MI355X"),
        "value": value, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": r["total_ms"] / args.steps,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": {"dn_prefill": "bf16", "gqa_prefill": "bf16", "q4_gemm": "f16",
                  "prefill_model": "f16"}.get(args.workload, "f32"),
        "data": ("synthetic (seeded normal logits, random generated ids)" if args.workload == "sample" else
                 "synthetic (seeded random Q4 codes, f16 scales and normal inputs)"
                 if args.workload.startswith("q4") or args.workload in ("lm_head", "decode_model", "prefill_model")
                 else "synthetic (seeded normal inputs, random-init state and f16 KV cache)"),
        "config": r["config"],
        "roofline": rl,
    }
    if args.workload == "stack":
        line["roofline"].update(stored_traffic(GQA_DECODE_SOURCES))
    for k in ("kernels", "step_frac_hbm", "graph_ms_per_step", "graph_step_frac_hbm", "eager_ms_per_step",
              "eager_event_ms_per_launch", "cold"):
        if k in r:
            line[k] = r[k]
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args.workload)
    if subs is not None:
        line["configs"] = subs
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
