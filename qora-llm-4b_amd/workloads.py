"""Seeded synthetic inputs for the mixer workloads (numpy, host memory).

Shapes are the QORA-4B mixer's (config.rs:42-97).  Distributions:
  - DeltaNet decode: activated q, k ~N(0,1) [16,128] (L2-normed by the op),
    v ~N(0,1) [32,128]; decay g = exp(-softplus(a) * exp(A_log)) with
    a ~N(0,1), dt_bias = 0, A_log = ln U(0.01, 0.1) per v head (drawn once),
    i.e. g = exp(-softplus(N(0,1)) * U(0.01,0.1)); beta = sigmoid(b),
    b ~N(0,1); z ~N(0,1); state ~N(0, 0.02); norm weight ~1+N(0,0.1) (f16).
  - GQA decode: q and gate ~N(0,1) interleaved per head, new k, v ~N(0,1),
    stored q/k norm weights ~N(0,0.1) (the (1+w) convention, gemv.rs:594),
    f16 K/V cache ~N(0,1).
  - DeltaNet prefill: raw qkv stream ~N(0,1) in bf16, depthwise conv weights
    ~N(0,0.5), a, b, A_log, dt_bias as decode, zero initial state.
  - GQA prefill: q, gate, k, v ~N(0,1) in bf16.
"""
from __future__ import annotations

import numpy as np

DN_QK, DN_V, DN_HD, DN_QKV, DN_VDIM = 16, 32, 128, 8192, 4096
GQA_H, GQA_KV, GQA_HD = 16, 4, 256


def f16_bits(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def f16_value(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_value(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def dn_params(rng: np.random.Generator) -> dict:
    return {
        "a_log": np.log(rng.uniform(0.01, 0.1, DN_V)).astype(np.float32),
        "dt_bias": np.zeros(DN_V, np.float32),
        "norm_w": f16_bits(1.0 + 0.1 * rng.standard_normal(DN_HD, dtype=np.float32)),
        "conv_w": (0.5 * rng.standard_normal((DN_QKV, 4), dtype=np.float32)),
    }


def dn_decode_workload(steps: int, batch: int = 1, seed: int = 0) -> dict:
    """Per-step activated inputs for `batch` sequences plus initial state."""
    rng = np.random.default_rng(seed)
    w = dn_params(rng)
    w["state0"] = (0.02 * rng.standard_normal((batch, DN_V, DN_HD, DN_HD), dtype=np.float32))
    w["qkv"] = rng.standard_normal((steps, batch, DN_QKV), dtype=np.float32)
    w["a"] = rng.standard_normal((steps, batch, DN_V), dtype=np.float32)
    w["b"] = rng.standard_normal((steps, batch, DN_V), dtype=np.float32)
    w["z"] = rng.standard_normal((steps, batch, DN_VDIM), dtype=np.float32)
    w["conv_buf0"] = np.zeros((batch, DN_QKV, 3), np.float32)
    return w


def gqa_decode_workload(pos: int, batch: int = 1, cap: int | None = None, seed: int = 1) -> dict:
    """One decode step at position `pos` (pos cached tokens) for `batch` sequences."""
    rng = np.random.default_rng(seed)
    cap = cap or pos + 1
    kc = np.zeros((batch, GQA_KV, cap, GQA_HD), np.uint16)
    vc = np.zeros_like(kc)
    kc[:, :, :pos] = f16_bits(rng.standard_normal((batch, GQA_KV, pos, GQA_HD), dtype=np.float32))
    vc[:, :, :pos] = f16_bits(rng.standard_normal((batch, GQA_KV, pos, GQA_HD), dtype=np.float32))
    return {
        "q_gate": rng.standard_normal((batch, GQA_H, 2 * GQA_HD), dtype=np.float32),
        "k_new": rng.standard_normal((batch, GQA_KV, GQA_HD), dtype=np.float32),
        "v_new": rng.standard_normal((batch, GQA_KV, GQA_HD), dtype=np.float32),
        "q_norm": f16_bits(0.1 * rng.standard_normal(GQA_HD, dtype=np.float32)),
        "k_norm": f16_bits(0.1 * rng.standard_normal(GQA_HD, dtype=np.float32)),
        "k_cache": kc, "v_cache": vc, "cap": cap, "pos": pos,
    }


def dn_prefill_workload(T: int, seed: int = 2) -> dict:
    rng = np.random.default_rng(seed)
    w = dn_params(rng)
    w["qkv"] = bf16_bits(rng.standard_normal((T, DN_QKV), dtype=np.float32))
    w["a"] = rng.standard_normal((T, DN_V), dtype=np.float32)
    w["b"] = rng.standard_normal((T, DN_V), dtype=np.float32)
    w["z"] = bf16_bits(rng.standard_normal((T, DN_VDIM), dtype=np.float32))
    w["state0"] = np.zeros((DN_V, DN_HD, DN_HD), np.float32)
    w["conv_buf0"] = np.zeros((DN_QKV, 3), np.float32)
    return w


def gqa_prefill_workload(S: int, seed: int = 3) -> dict:
    rng = np.random.default_rng(seed)
    return {
        "q_gate": bf16_bits(rng.standard_normal((S, GQA_H, 2 * GQA_HD), dtype=np.float32)),
        "k": bf16_bits(rng.standard_normal((S, GQA_KV, GQA_HD), dtype=np.float32)),
        "v": bf16_bits(rng.standard_normal((S, GQA_KV, GQA_HD), dtype=np.float32)),
        "q_norm": f16_bits(0.1 * rng.standard_normal(GQA_HD, dtype=np.float32)),
        "k_norm": f16_bits(0.1 * rng.standard_normal(GQA_HD, dtype=np.float32)),
    }


# ---- Q4 projections (gemv.rs:29-34 layout) -------------------------------------
# (k input rows, n outputs) of the QORA-4B projections around the mixer
# (config.rs:42-79: hidden 2560, intermediate 9216).
Q4_PROJ_SHAPES = {
    "in_proj_qkv": (2560, 8192), "in_proj_z": (2560, 4096), "in_proj_a": (2560, 32),
    "in_proj_b": (2560, 32), "out_proj": (4096, 2560), "q_proj": (2560, 8192),
    "k_proj": (2560, 1024), "v_proj": (2560, 1024), "o_proj": (4096, 2560),
    "gate_proj": (2560, 9216), "up_proj": (2560, 9216), "down_proj": (9216, 2560),
}


def q4_dequant(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """W [k, n] f32 from Q4 codes: scale(row, n // 32) * (q - 8), low nibble = even column."""
    packed = np.asarray(packed, np.uint8)
    k, half = packed.shape
    q = np.empty((k, 2 * half), np.int32)
    q[:, 0::2] = packed & 0x0F
    q[:, 1::2] = packed >> 4
    s = f16_value(scales).astype(np.float32)
    return np.repeat(s, 32, axis=1) * (q - 8).astype(np.float32)


def q4_tile(n: int) -> int:
    """Column-tile width of the device layout (QM_Q4_TILE)."""
    return 8 if n < 4096 else 16


def q4_device_layout(packed: np.ndarray, scales: np.ndarray):
    """Reference layout -> device layout: codes [n/T, k, T/2], gscales [n/32, k]."""
    packed = np.asarray(packed, np.uint8)
    k, half = packed.shape
    t = q4_tile(2 * half)
    codes = np.ascontiguousarray(packed.reshape(k, 2 * half // t, t // 2).transpose(1, 0, 2))
    return codes, np.ascontiguousarray(np.asarray(scales, np.uint16).T)


def q4_random_weight(k: int, n: int, rng: np.random.Generator, scale: float = 0.006):
    """Valid Q4 codes and f16 scales of the size a quantized N(0, 0.02)
    weight has (absmax / 7 of 32 draws ~ 0.006)."""
    packed = rng.integers(0, 256, (k, n // 2), dtype=np.uint8)
    scales = f16_bits(scale * (1.0 + 0.2 * rng.standard_normal((k, n // 32), dtype=np.float32)))
    return packed, scales


def q4_gemv_workload(k: int, n: int, seed: int = 5) -> dict:
    rng = np.random.default_rng(seed)
    packed, scales = q4_random_weight(k, n, rng)
    return {"x": rng.standard_normal(k, dtype=np.float32), "packed": packed, "scales": scales}
