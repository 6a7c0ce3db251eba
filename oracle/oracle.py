"""numpy front end of the CPU oracle (liboracle.so, built from qora_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product library.  Each wrapper
calls the C restatement of one reference function (citations in
qora_oracle.h / qora_oracle.c).
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"

UPDATE_SCALAR, UPDATE_AVX512, UPDATE_AVX512_EMUL, UPDATE_AUTO = 0, 1, 2, 3


class OrConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "num_qk_heads", "num_v_heads", "dn_head_dim", "conv_kernel",
        "num_heads", "num_kv_heads", "attn_head_dim", "rope_dim")]


def config(num_qk_heads=16, num_v_heads=32, dn_head_dim=128, conv_kernel=4,
           num_heads=16, num_kv_heads=4, attn_head_dim=256, rope_dim=64) -> OrConfig:
    """Qor4bConfig::default_4b mixer dims (config.rs:42-97), overridable for tiny cases."""
    return OrConfig(num_qk_heads, num_v_heads, dn_head_dim, conv_kernel,
                    num_heads, num_kv_heads, attn_head_dim, rope_dim)


_P, _I32, _F32 = C.c_void_p, C.c_int32, C.c_float
_SIG = {
    "or_f16_to_f32": ([C.c_uint16], _F32),
    "or_f32_to_f16": ([_F32], C.c_uint16),
    "or_bf16_to_f32": ([C.c_uint16], _F32),
    "or_f32_to_bf16": ([_F32], C.c_uint16),
    "or_silu": ([_F32], _F32),
    "or_softplus": ([_F32], _F32),
    "or_l2_normalize": ([_P, _I32], None),
    "or_softmax_raw": ([_P, _I32], None),
    "or_rms_norm": ([_P, _I32, _P, _P], None),
    "or_per_head_rms_norm": ([_P, _I32, _I32, _P], None),
    "or_apply_partial_rope": ([_P, _I32, _I32, _P, _P, _I32, _I32], None),
    "or_rope_table": ([C.c_double, _I32, _I32, _P, _P], None),
    "or_deltanet_head_update_scalar": ([_P, _P, _P, _P, _F32, _F32, _I32, _P], None),
    "or_deltanet_head_update_avx512": ([_P, _P, _P, _P, _F32, _F32, _I32, _P], _I32),
    "or_deltanet_head_update_avx512_emul": ([_P, _P, _P, _P, _F32, _F32, _I32, _P], None),
    "or_has_avx512": ([], _I32),
    "or_conv1d_step": ([_I32, _I32, _P, _P, _P, _P], None),
    "or_deltanet_decode_step": ([C.POINTER(OrConfig), _P, _I32, _P, _P, _P, _P, _P, _P, _P, _P,
                                 _P, _P, _I32], None),
    "or_deltanet_decode_step_mt": ([C.POINTER(OrConfig), _P, _I32, _P, _P, _P, _P, _P, _P, _P, _P,
                                    _P, _P, _I32, _I32], None),
    "or_deltanet_prefill": ([C.POINTER(OrConfig), _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                             _P], None),
    "or_attn_decode_step": ([C.POINTER(OrConfig), _P, _P, _P, _P, _P, _P, _P, _I32, _P, _P, _I32,
                             _I32, _P, _I32], _I32),
    "or_attn_prefill": ([C.POINTER(OrConfig), _I32, _P, _P, _P, _P, _P, _P, _P, _I32, _P, _P, _P,
                         _P, _I32, _I32], _I32),
    "or_q4_quantize": ([_P, _I32, _I32, _P, _P], None),
    "or_q4_gemv": ([_P, _P, _P, _I32, _I32, _P], None),
    "or_q4_gemm": ([_P, _I32, _P, _P, _I32, _I32, _P, _I32], None),
    "or_q4_gate_up": ([_P, _P, _P, _P, _P, _I32, _I32, _P], None),
    "or_q4_lm_head": ([_P, _P, _P, _I32, _I32, _P, _I32], None),
    "or_q4_embed": ([_P, _P, _I32, _I32, _P], None),
    "or_rng_next_f32": ([_P], C.c_float),
    "or_apply_repetition_penalty": ([_P, _I32, _P, _I32, C.c_float], None),
    "or_apply_presence_penalty": ([_P, _I32, _P, _I32, C.c_float], None),
    "or_sample_top_k": ([_P, _I32, C.c_float, C.c_float, _I32, _P, _I32, _P, _P], _I32),
}

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
        _lib = C.CDLL(str(LIB_PATH))
        for name, (args, res) in _SIG.items():
            f = getattr(_lib, name)
            f.argtypes = args
            f.restype = res
    return _lib


def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32)


def _ptr(a):
    return None if a is None else a.ctypes.data


# ---- conversions -------------------------------------------------------------
def f16_bits(x) -> np.ndarray:
    """f32 -> IEEE f16 bit patterns (RNE), via the oracle's converter."""
    x = _f32(x)
    f = lib().or_f32_to_f16
    return np.array([f(float(v)) for v in x.ravel()], np.uint16).reshape(x.shape)


def f16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, np.uint16)
    f = lib().or_f16_to_f32
    return np.array([f(int(v)) for v in h.ravel()], np.float32).reshape(h.shape)


def has_avx512() -> bool:
    return bool(lib().or_has_avx512())


# ---- helpers -----------------------------------------------------------------
def silu(x: float) -> float:
    return lib().or_silu(x)


def softplus(x: float) -> float:
    return lib().or_softplus(x)


def l2_normalize(x) -> np.ndarray:
    x = _f32(x).copy()
    lib().or_l2_normalize(x.ctypes.data, x.size)
    return x


def softmax_raw(x) -> np.ndarray:
    x = _f32(x).copy()
    lib().or_softmax_raw(x.ctypes.data, x.size)
    return x


def rms_norm(x, gamma_f16) -> np.ndarray:
    x = _f32(x)
    g = np.ascontiguousarray(gamma_f16, np.uint16)
    out = np.empty_like(x)
    lib().or_rms_norm(x.ctypes.data, x.size, g.ctypes.data, out.ctypes.data)
    return out


def per_head_rms_norm(x, num_heads, head_dim, gamma_f16) -> np.ndarray:
    x = _f32(x).copy()
    g = np.ascontiguousarray(gamma_f16, np.uint16)
    lib().or_per_head_rms_norm(x.ctypes.data, num_heads, head_dim, g.ctypes.data)
    return x


def apply_partial_rope(x, num_heads, head_dim, cos, sin, rotary_dim, position) -> np.ndarray:
    x = _f32(x).copy()
    cos, sin = _f32(cos), _f32(sin)
    lib().or_apply_partial_rope(x.ctypes.data, num_heads, head_dim, cos.ctypes.data,
                                sin.ctypes.data, rotary_dim, position)
    return x


def rope_table(max_pos, theta=1e7, rope_dim=64):
    cos = np.empty((max_pos, rope_dim // 2), np.float32)
    sin = np.empty_like(cos)
    lib().or_rope_table(theta, rope_dim, max_pos, cos.ctypes.data, sin.ctypes.data)
    return cos, sin


def head_update(s, q, k, v, alpha, beta, kind=UPDATE_SCALAR):
    """One v-head delta-rule update; returns (S', y)."""
    s = _f32(s).copy()
    q, k, v = _f32(q), _f32(k), _f32(v)
    hd = q.size
    y = np.empty(hd, np.float32)
    args = (s.ctypes.data, q.ctypes.data, k.ctypes.data, v.ctypes.data, alpha, beta, hd, y.ctypes.data)
    if kind == UPDATE_SCALAR:
        lib().or_deltanet_head_update_scalar(*args)
    elif kind == UPDATE_AVX512:
        if lib().or_deltanet_head_update_avx512(*args) != 0:
            raise RuntimeError("host has no AVX-512F")
    else:
        lib().or_deltanet_head_update_avx512_emul(*args)
    return s, y


def conv1d_step(conv_buf, conv_w, x):
    """gemv.rs:744-769: returns the pre-SiLU conv output; conv_buf shifts in place."""
    assert conv_buf.dtype == np.float32 and conv_buf.flags.c_contiguous
    conv_w, x = _f32(conv_w), _f32(x)
    n, ks = conv_w.shape
    out = np.empty(n, np.float32)
    lib().or_conv1d_step(n, ks, conv_buf.ctypes.data, conv_w.ctypes.data, x.ctypes.data,
                         out.ctypes.data)
    return out


# ---- layer slices --------------------------------------------------------------
def deltanet_decode_step(cfg, qkv, a, b, z, conv_w, a_log, dt_bias, norm_w_f16, state,
                         conv_buf=None, preact=False, kind=UPDATE_AUTO, nthreads=1):
    """gemv.rs:744-883.  state / conv_buf are updated in place; returns out.
    nthreads > 1 runs the v-head loop in parallel (the reference's loop at
    gemv.rs:817 is serial); the result does not depend on it."""
    qkv, a, b, z = _f32(qkv), _f32(a), _f32(b), _f32(z)
    conv_w, a_log, dt_bias = _f32(conv_w), _f32(a_log), _f32(dt_bias)
    nw = np.ascontiguousarray(norm_w_f16, np.uint16)
    assert state.dtype == np.float32 and state.flags.c_contiguous
    if preact:
        assert conv_buf is not None and conv_buf.dtype == np.float32 and conv_buf.flags.c_contiguous
    out = np.empty(cfg.num_v_heads * cfg.dn_head_dim, np.float32)
    lib().or_deltanet_decode_step_mt(C.byref(cfg), qkv.ctypes.data, int(preact), _ptr(conv_buf),
                                     conv_w.ctypes.data, a.ctypes.data, b.ctypes.data,
                                     a_log.ctypes.data, dt_bias.ctypes.data, z.ctypes.data,
                                     nw.ctypes.data, state.ctypes.data, out.ctypes.data, kind,
                                     int(nthreads))
    return out


def deltanet_prefill(cfg, qkv_all, a_all, b_all, z_all, conv_w, a_log, dt_bias, norm_w_f16,
                     state, conv_buf):
    """gemv.rs:1119-1219.  state / conv_buf updated in place; returns out [T, v_dim]."""
    qkv_all, a_all, b_all, z_all = _f32(qkv_all), _f32(a_all), _f32(b_all), _f32(z_all)
    conv_w, a_log, dt_bias = _f32(conv_w), _f32(a_log), _f32(dt_bias)
    nw = np.ascontiguousarray(norm_w_f16, np.uint16)
    T = qkv_all.shape[0]
    out = np.empty((T, cfg.num_v_heads * cfg.dn_head_dim), np.float32)
    lib().or_deltanet_prefill(C.byref(cfg), T, qkv_all.ctypes.data, a_all.ctypes.data,
                              b_all.ctypes.data, z_all.ctypes.data, conv_buf.ctypes.data,
                              conv_w.ctypes.data, a_log.ctypes.data, dt_bias.ctypes.data,
                              nw.ctypes.data, state.ctypes.data, out.ctypes.data)
    return out


def attn_decode_step(cfg, q_gate, k_new, v_new, q_norm_f16, k_norm_f16, cos, sin, k_cache,
                     v_cache, seq_len, round_kv_f16=False, nthreads=1):
    """gemv.rs:927-1011.  k_cache/v_cache [>= seq_len+1, KV, D] f32, row seq_len written."""
    q_gate, k_new, v_new = _f32(q_gate), _f32(k_new), _f32(v_new)
    qn = np.ascontiguousarray(q_norm_f16, np.uint16)
    kn = np.ascontiguousarray(k_norm_f16, np.uint16)
    cos, sin = _f32(cos), _f32(sin)
    assert k_cache.dtype == np.float32 and k_cache.flags.c_contiguous
    assert v_cache.dtype == np.float32 and v_cache.flags.c_contiguous
    out = np.empty(cfg.num_heads * cfg.attn_head_dim, np.float32)
    st = lib().or_attn_decode_step(C.byref(cfg), q_gate.ctypes.data, k_new.ctypes.data,
                                   v_new.ctypes.data, qn.ctypes.data, kn.ctypes.data,
                                   cos.ctypes.data, sin.ctypes.data, cos.shape[0],
                                   k_cache.ctypes.data, v_cache.ctypes.data, seq_len,
                                   int(round_kv_f16), out.ctypes.data, nthreads)
    if st != 0:
        raise IndexError("RoPE position beyond table")
    return out


def attn_prefill(cfg, q_gate_all, k_all, v_all, q_norm_f16, k_norm_f16, cos, sin, rows=None,
                 nthreads=1):
    """gemv.rs:1364-1444.  Returns (out [S, H*D], k_cache [S,KV,D], v_cache)."""
    q_gate_all, k_all, v_all = _f32(q_gate_all), _f32(k_all), _f32(v_all)
    qn = np.ascontiguousarray(q_norm_f16, np.uint16)
    kn = np.ascontiguousarray(k_norm_f16, np.uint16)
    cos, sin = _f32(cos), _f32(sin)
    S = q_gate_all.shape[0]
    H, KV, D = cfg.num_heads, cfg.num_kv_heads, cfg.attn_head_dim
    out = np.zeros((S, H * D), np.float32)
    kc = np.empty((S, KV, D), np.float32)
    vc = np.empty((S, KV, D), np.float32)
    r = None if rows is None else np.ascontiguousarray(rows, np.int32)
    st = lib().or_attn_prefill(C.byref(cfg), S, q_gate_all.ctypes.data, k_all.ctypes.data,
                               v_all.ctypes.data, qn.ctypes.data, kn.ctypes.data, cos.ctypes.data,
                               sin.ctypes.data, cos.shape[0], kc.ctypes.data, vc.ctypes.data,
                               out.ctypes.data, _ptr(r), 0 if r is None else r.size, nthreads)
    if st != 0:
        raise IndexError("RoPE position beyond table")
    return out, kc, vc


# ---- Q4 projections ------------------------------------------------------------
def q4_quantize(w):
    """convert.rs:437-467.  w f32 [k, n] (n % 32 == 0) -> (packed u8 [k, n/2], scales f16 bits [k, n/32])."""
    w = _f32(w)
    k, n = w.shape
    assert n % 32 == 0
    packed = np.empty((k, n // 2), np.uint8)
    scales = np.empty((k, n // 32), np.uint16)
    lib().or_q4_quantize(w.ctypes.data, k, n, packed.ctypes.data, scales.ctypes.data)
    return packed, scales


def q4_gemv(x, packed, scales):
    """gemv.rs:412-445 over all k rows: y = x @ W."""
    x = _f32(x)
    packed = np.ascontiguousarray(packed, np.uint8)
    scales = np.ascontiguousarray(scales, np.uint16)
    k, n = packed.shape[0], packed.shape[1] * 2
    assert x.size == k
    y = np.empty(n, np.float32)
    lib().or_q4_gemv(x.ctypes.data, packed.ctypes.data, scales.ctypes.data, k, n, y.ctypes.data)
    return y


def q4_gemm(x, packed, scales, nthreads=8):
    """gemv.rs:529-542: rows of x [m, k] through gemv_q4_inner."""
    x = _f32(x)
    packed = np.ascontiguousarray(packed, np.uint8)
    scales = np.ascontiguousarray(scales, np.uint16)
    k, n = packed.shape[0], packed.shape[1] * 2
    m = x.shape[0]
    assert x.shape[1] == k
    y = np.empty((m, n), np.float32)
    lib().or_q4_gemm(x.ctypes.data, m, packed.ctypes.data, scales.ctypes.data, k, n, y.ctypes.data,
                     nthreads)
    return y


def q4_gate_up(x, g_packed, g_scales, u_packed, u_scales):
    """gemv.rs:469-526: silu(x @ Wg) * (x @ Wu)."""
    x = _f32(x)
    gp, up = (np.ascontiguousarray(a, np.uint8) for a in (g_packed, u_packed))
    gs, us = (np.ascontiguousarray(a, np.uint16) for a in (g_scales, u_scales))
    k, n = gp.shape[0], gp.shape[1] * 2
    out = np.empty(n, np.float32)
    lib().or_q4_gate_up(x.ctypes.data, gp.ctypes.data, gs.ctypes.data, up.ctypes.data,
                        us.ctypes.data, k, n, out.ctypes.data)
    return out


# ---- vocabulary side ---------------------------------------------------------
def q4_lm_head(x, packed, scales, nthreads=8):
    """gemv.rs:678-708: logits[v] = x . row v of the vocab-major Q4 embedding
    (packed [vocab, hidden/2], scales [vocab, hidden/32])."""
    x = _f32(x)
    packed = np.ascontiguousarray(packed, np.uint8)
    scales = np.ascontiguousarray(scales, np.uint16)
    vocab, hidden = packed.shape[0], packed.shape[1] * 2
    assert x.size == hidden
    out = np.empty(vocab, np.float32)
    lib().or_q4_lm_head(x.ctypes.data, packed.ctypes.data, scales.ctypes.data, vocab, hidden,
                        out.ctypes.data, nthreads)
    return out


def q4_embed(packed, scales, token_id):
    """gemv.rs:544-563: the dequantized embedding row of token_id."""
    packed = np.ascontiguousarray(packed, np.uint8)
    scales = np.ascontiguousarray(scales, np.uint16)
    vocab, hidden = packed.shape[0], packed.shape[1] * 2
    assert 0 <= token_id < vocab
    out = np.empty(hidden, np.float32)
    lib().or_q4_embed(packed.ctypes.data, scales.ctypes.data, hidden, int(token_id), out.ctypes.data)
    return out


# ---- sampling ----------------------------------------------------------------
def rng_next_f32(state: np.ndarray) -> float:
    """generate.rs:46-54; state is a uint64 array of one element, advanced in place."""
    assert state.dtype == np.uint64 and state.size == 1
    return lib().or_rng_next_f32(state.ctypes.data)


def apply_penalties(logits, generated, repetition_penalty, presence_penalty):
    """generate.rs:58-82, repetition then presence (generate.rs:194-195); returns a copy."""
    out = _f32(logits).copy()
    g = np.ascontiguousarray(generated, np.int32)
    lib().or_apply_repetition_penalty(out.ctypes.data, out.size, g.ctypes.data, g.size, repetition_penalty)
    lib().or_apply_presence_penalty(out.ctypes.data, out.size, g.ctypes.data, g.size, presence_penalty)
    return out


def sample_top_k(logits, temperature, top_p, top_k, state, wgpu=False):
    """sample_token_top_k (generate.rs:334-384, or gpu_inference.rs:867-906 with
    wgpu): returns (token, sorted top-k ids, their probabilities); state (uint64
    array of one element) is advanced in place when a draw is made."""
    x = _f32(logits)
    k = 1 if temperature <= 0 else (min(top_k, x.size) if top_k > 0 else x.size)
    ids = np.zeros(k, np.int32)
    probs = np.zeros(k, np.float32)
    tok = lib().or_sample_top_k(x.ctypes.data, x.size, temperature, top_p, top_k, state.ctypes.data,
                                int(wgpu), ids.ctypes.data, probs.ctypes.data)
    return tok, ids, probs
