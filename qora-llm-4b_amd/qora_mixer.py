"""ctypes binding of libqora_mixer.so (the C ABI in include/qora_mixer.h).

This is the Python-side caller of the MI355X mixer library, used by the
tests and the benchmark.  It is a thin, typed mirror of the C entry points:
device buffers are plain integer addresses owned by `DeviceBuffer`, arrays
cross the boundary as numpy arrays, and every non-zero status raises
`MixerError` carrying the library's status code and message.  There is no
fallback path: if the library or its code objects are missing, creating a
`Context` fails loudly.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent
LIB_DIR = PKG_DIR / "lib"
LIB_PATH = LIB_DIR / "libqora_mixer.so"

QM_OK = 0
STATUS_NAMES = {
    0: "QM_OK", 1: "QM_ERR_NO_DEVICE", 2: "QM_ERR_CODE_OBJECT", 3: "QM_ERR_INVALID_ARG",
    4: "QM_ERR_SHAPE", 5: "QM_ERR_ROPE_RANGE", 6: "QM_ERR_CAPACITY", 7: "QM_ERR_HIP",
    8: "QM_ERR_OUT_OF_MEMORY", 9: "QM_ERR_WORKSPACE",
}
QM_DN_POSTACT, QM_DN_PREACT = 0, 1
QM_F32, QM_F16, QM_BF16 = 0, 1, 2
QM_OPT_DN_DECODE_THREADS, QM_OPT_GQA_DECODE_CHUNK, QM_OPT_GQA_PREFILL_ORDER = 1, 2, 3

# Mixer shape (config.rs:42-97).
DN_QK_HEADS, DN_V_HEADS, DN_HD, DN_CONV_K = 16, 32, 128, 4
DN_QKV_DIM, DN_V_DIM = 8192, 4096
GQA_HEADS, GQA_KV_HEADS, GQA_HD, GQA_ROT = 16, 4, 256, 64
ROPE_THETA = 10_000_000.0


class QmQ4Out(C.Structure):
    _fields_ = [("n", C.c_int32), ("codes_dev", C.c_void_p), ("gscales_dev", C.c_void_p),
                ("y_dev", C.c_void_p), ("residual_dev", C.c_void_p)]


QM_SAMPLE_WGPU = 1


class QmSampleParams(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_int32),
                ("repetition_penalty", C.c_float), ("presence_penalty", C.c_float),
                ("banned_id", C.c_int32), ("flags", C.c_int32)]


class QmConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "num_qk_heads", "num_v_heads", "dn_head_dim", "conv_kernel",
        "num_heads", "num_kv_heads", "attn_head_dim", "rope_dim")]


class MixerError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(code, code)}: {message}")
        self.code = code
        self.message = message


_P, _I32, _I64, _U64 = C.c_void_p, C.c_int32, C.c_int64, C.c_uint64

# name -> argtypes (restype is int32 unless listed in _RESTYPES)
_SIGNATURES = {
    "qm_default_config": [C.POINTER(QmConfig)],
    "qm_create": [C.POINTER(_P), C.POINTER(QmConfig), C.c_char_p, _I32],
    "qm_destroy": [_P],
    "qm_status_string": [_I32],
    "qm_last_error": [_P],
    "qm_device_count": [C.POINTER(_I32)],
    "qm_reserve": [_P, _I32, _I32, _I32],
    "qm_set_option": [_P, _I32, _I64],
    "qm_alloc": [_P, _U64, C.POINTER(_P)],
    "qm_free": [_P, _P],
    "qm_memcpy_h2d": [_P, _P, _P, _U64, _P],
    "qm_memcpy_d2h": [_P, _P, _P, _U64, _P],
    "qm_memcpy_d2d": [_P, _P, _P, _U64, _P],
    "qm_memset": [_P, _P, _I32, _U64, _P],
    "qm_stream_create": [_P, C.POINTER(_P)],
    "qm_stream_destroy": [_P, _P],
    "qm_sync": [_P, _P],
    "qm_event_create": [_P, C.POINTER(_P)],
    "qm_event_destroy": [_P, _P],
    "qm_event_record": [_P, _P, _P],
    "qm_event_elapsed_ms": [_P, _P, _P, C.POINTER(C.c_float)],
    "qm_graph_begin": [_P, _P],
    "qm_graph_end": [_P, _P, C.POINTER(_P)],
    "qm_graph_launch": [_P, _P, _P],
    "qm_graph_destroy": [_P, _P],
    "qm_rope_table": [C.c_double, _I32, _I32, _P, _P],
    "qm_fill_normal": [_P, _P, _I32, _U64, C.c_float, C.c_float, _U64, _P],
    "qm_deltanet_decode": [_P, _P, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _P],
    "qm_deltanet_prefill": [_P, _P, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P],
    "qm_gqa_decode": [_P, _P, _I32, _P, _P, _P, _P, _P, _P, _P, _I32, _P, _I32, _P, _P, _I64, _P],
    "qm_gqa_decode_noalloc": [_P, _P, _I32, _P, _P, _P, _P, _P, _P, _P, _I32, _P, _I32, _P, _P, _I64, _P],
    "qm_gqa_prefill": [_P, _P, _I32, _P, _P, _P, _P, _P, _P, _P, _I32, _P, _P, _I64, _P],
    "qm_q4_repack": [_P, _P, _I32, _I32, _P, _P, _P, _P],
    "qm_q4_gemv": [_P, _P, _I32, _I32, _P, _P, _P, _P],
    "qm_q4_gemv_multi": [_P, _P, _I32, _P, _P, _I32, _P],
    "qm_q4_gemv_multi_conv": [_P, _P, _I32, _P, _P, _I32, _P, _P, _P],
    "qm_q4_gate_up": [_P, _P, _I32, _I32, _P, _P, _P, _P, _P, _P, _P],
    "qm_rms_norm_f16": [_P, _P, _I32, _I32, _P, _P, _P],
    "qm_q4_gemm": [_P, _P, _I32, _I32, _I32, _P, _I32, _P, _P, _P, _P, _P],
    "qm_q4_gemm_gate_up": [_P, _P, _I32, _I32, _I32, _P, _I32, _P, _P, _P, _P, _P],
    "qm_q4_lm_head": [_P, _P, _I32, _I32, _P, _P, _P, _P, _P],
    "qm_q4_embed": [_P, _P, _I32, _I32, _I32, _P, _P, _P, _P],
    "qm_sample": [_P, _P, _I32, _P, _P, _I32, C.POINTER(QmSampleParams), _P, _P, _P, _P],
}
_RESTYPES = {"qm_default_config": None, "qm_status_string": C.c_char_p, "qm_last_error": C.c_char_p}

_lib = None


def load_library(path: str | os.PathLike | None = None) -> C.CDLL:
    """Load libqora_mixer.so and declare every exported entry point."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise FileNotFoundError(f"{p} is not built; run `python qora-llm-4b_amd/build.py`")
    lib = C.CDLL(str(p))
    for name, argtypes in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, _I32)
    if path is None:
        _lib = lib
    return lib


def default_config() -> QmConfig:
    cfg = QmConfig()
    load_library().qm_default_config(C.byref(cfg))
    return cfg


def rope_table(max_pos: int, theta: float = ROPE_THETA, rope_dim: int = GQA_ROT):
    """convert.rs:161-176 tables, shape [max_pos, rope_dim/2] float32."""
    cos = np.empty((max_pos, rope_dim // 2), np.float32)
    sin = np.empty_like(cos)
    st = load_library().qm_rope_table(theta, rope_dim, max_pos, cos.ctypes.data, sin.ctypes.data)
    if st != QM_OK:
        raise MixerError(st, "qm_rope_table")
    return cos, sin


def device_count() -> int:
    n = _I32(0)
    load_library().qm_device_count(C.byref(n))
    return int(n.value)


def _addr(x) -> int | None:
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    return int(x)


class DeviceBuffer:
    """A device allocation made through qm_alloc; freed on close()/GC."""

    def __init__(self, ctx: "Context", nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = _P(0)
        ctx._check(ctx.lib.qm_alloc(ctx.h, self.nbytes, C.byref(p)))
        self.ptr = int(p.value)

    def offset(self, nbytes: int) -> int:
        if not 0 <= nbytes <= self.nbytes:
            raise ValueError("offset outside the buffer")
        return self.ptr + int(nbytes)

    def close(self):
        if self.ptr and self.ctx.h:
            self.ctx.lib.qm_free(self.ctx.h, self.ptr)
        self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Context:
    """One qm_context on one device (not thread-safe, one stream at a time)."""

    def __init__(self, device: int = 0, code_object_dir: str | None = None):
        """code_object_dir: directory of the qm_*.hsaco files; default is the
        QORA_MIXER_CODE_OBJECTS environment variable, else the library's own
        directory."""
        self.lib = load_library()
        code_object_dir = code_object_dir or os.environ.get("QORA_MIXER_CODE_OBJECTS") or None
        h = _P(0)
        cdir = str(code_object_dir).encode() if code_object_dir else None
        st = self.lib.qm_create(C.byref(h), None, cdir, device)
        if st != QM_OK:
            raise MixerError(st, self.lib.qm_last_error(None).decode())
        self.h = h.value
        self.stream = None  # the context's own stream

    def close(self):
        if getattr(self, "h", None):
            self.lib.qm_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, st: int):
        if st != QM_OK:
            raise MixerError(st, self.lib.qm_last_error(self.h).decode())

    def last_error(self) -> str:
        return self.lib.qm_last_error(self.h).decode()

    # ---- plumbing -------------------------------------------------------
    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def upload(self, arr: np.ndarray, buf: DeviceBuffer | None = None) -> DeviceBuffer:
        arr = np.ascontiguousarray(arr)
        if buf is None:
            buf = self.alloc(max(arr.nbytes, 1))
        elif buf.nbytes < arr.nbytes:
            raise ValueError("buffer too small")
        self._check(self.lib.qm_memcpy_h2d(self.h, buf.ptr, arr.ctypes.data, arr.nbytes, self.stream))
        return buf

    def upload_to(self, addr: int, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        self._check(self.lib.qm_memcpy_h2d(self.h, int(addr), arr.ctypes.data, arr.nbytes, self.stream))

    def download(self, src, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype)
        self._check(self.lib.qm_memcpy_d2h(self.h, out.ctypes.data, _addr(src), out.nbytes, self.stream))
        return out

    def copy(self, dst, src, nbytes: int):
        self._check(self.lib.qm_memcpy_d2d(self.h, _addr(dst), _addr(src), int(nbytes), self.stream))

    def memset(self, dst, value: int, nbytes: int):
        self._check(self.lib.qm_memset(self.h, _addr(dst), value, int(nbytes), self.stream))

    def fill_normal(self, dst, dtype: int, count: int, mean: float, std: float, seed: int):
        self._check(self.lib.qm_fill_normal(self.h, _addr(dst), dtype, int(count), mean, std, int(seed), self.stream))

    def sync(self):
        self._check(self.lib.qm_sync(self.h, self.stream))

    def reserve(self, max_batch: int, max_kv_len: int = 0, max_prefill_tokens: int = 0):
        self._check(self.lib.qm_reserve(self.h, max_batch, max_kv_len, max_prefill_tokens))

    def set_option(self, option: int, value: int):
        self._check(self.lib.qm_set_option(self.h, option, int(value)))

    def event(self) -> "Event":
        return Event(self)

    def graph_begin(self):
        self._check(self.lib.qm_graph_begin(self.h, self.stream))

    def graph_end(self) -> "Graph":
        g = _P(0)
        self._check(self.lib.qm_graph_end(self.h, self.stream, C.byref(g)))
        return Graph(self, g.value)

    # ---- mixer ops --------------------------------------------------------
    def deltanet_decode(self, batch, flags, qkv, conv_buf, conv_w, a, b, a_log, dt_bias, z,
                        norm_w, state, out, state_stride=DN_V_HEADS * DN_HD * DN_HD):
        self._check(self.lib.qm_deltanet_decode(
            self.h, self.stream, batch, flags, _addr(qkv), _addr(conv_buf), _addr(conv_w),
            _addr(a), _addr(b), _addr(a_log), _addr(dt_bias), _addr(z), _addr(norm_w),
            _addr(state), state_stride, _addr(out)))

    def deltanet_prefill(self, seq_len, qkv, conv_buf, conv_w, a, b, a_log, dt_bias, z, norm_w,
                         state, out):
        self._check(self.lib.qm_deltanet_prefill(
            self.h, self.stream, seq_len, _addr(qkv), _addr(conv_buf), _addr(conv_w), _addr(a),
            _addr(b), _addr(a_log), _addr(dt_bias), _addr(z), _addr(norm_w), _addr(state),
            _addr(out)))

    def gqa_decode(self, batch, q_gate, k_new, v_new, q_norm, k_norm, rope_cos, rope_sin,
                   rope_len, pos, max_pos, k_cache, v_cache, cap, out):
        self._check(self.lib.qm_gqa_decode(
            self.h, self.stream, batch, _addr(q_gate), _addr(k_new), _addr(v_new), _addr(q_norm),
            _addr(k_norm), _addr(rope_cos), _addr(rope_sin), rope_len, _addr(pos), max_pos,
            _addr(k_cache), _addr(v_cache), cap, _addr(out)))

    def gqa_decode_noalloc(self, batch, q_gate, k_new, v_new, q_norm, k_norm, rope_cos, rope_sin,
                           rope_len, pos, max_pos, k_cache, v_cache, cap, out):
        """qm_gqa_decode with its partials in the device's fixed scratch array (no allocation)."""
        self._check(self.lib.qm_gqa_decode_noalloc(
            self.h, self.stream, batch, _addr(q_gate), _addr(k_new), _addr(v_new), _addr(q_norm),
            _addr(k_norm), _addr(rope_cos), _addr(rope_sin), rope_len, _addr(pos), max_pos,
            _addr(k_cache), _addr(v_cache), cap, _addr(out)))

    def gqa_prefill(self, seq_len, q_gate, k, v, q_norm, k_norm, rope_cos, rope_sin, rope_len,
                    k_cache, v_cache, cap, out):
        self._check(self.lib.qm_gqa_prefill(
            self.h, self.stream, seq_len, _addr(q_gate), _addr(k), _addr(v), _addr(q_norm),
            _addr(k_norm), _addr(rope_cos), _addr(rope_sin), rope_len, _addr(k_cache),
            _addr(v_cache), cap, _addr(out)))

    def q4_repack(self, k, n, packed, scales, codes, gscales):
        """Reference Q4Weight layout (packed [k][n/2], scales [k][n/32]) -> the
        tile-major device layout (codes [n/T][k][T/2], gscales [n/32][k], T = 8 if n < 4096 else 16)."""
        self._check(self.lib.qm_q4_repack(self.h, self.stream, k, n, _addr(packed), _addr(scales),
                                          _addr(codes), _addr(gscales)))

    def q4_gemv(self, k, n, x, codes, gscales, y):
        """y[n] = x[k] @ W for a Q4 weight in the device layout."""
        self._check(self.lib.qm_q4_gemv(self.h, self.stream, k, n, _addr(x), _addr(codes),
                                        _addr(gscales), _addr(y)))

    def q4_gemv_multi(self, k, x, outs, norm_w=None, conv_buf=None, conv_w=None):
        """outs: [(n, codes, gscales, y) or (n, codes, gscales, y, residual), ...]
        (1..4 weights sharing x); norm_w: optional f16 [k] RMSNorm weight.  With
        conv_buf / conv_w, outs[0] gets the DeltaNet conv1d step + SiLU."""
        arr = (QmQ4Out * len(outs))(*[
            QmQ4Out(o[0], _addr(o[1]), _addr(o[2]), _addr(o[3]), _addr(o[4]) if len(o) > 4 else None)
            for o in outs])
        if conv_buf is None and conv_w is None:
            self._check(self.lib.qm_q4_gemv_multi(self.h, self.stream, k, _addr(x), _addr(norm_w), len(outs), arr))
        else:
            self._check(self.lib.qm_q4_gemv_multi_conv(self.h, self.stream, k, _addr(x), _addr(norm_w), len(outs),
                                                       arr, _addr(conv_buf), _addr(conv_w)))

    def rms_norm_f16(self, m, k, x, norm_w, out):
        """out f16 [m, k] = rms_norm(x, norm_w) per row (or plain f16 if norm_w is None)."""
        self._check(self.lib.qm_rms_norm_f16(self.h, self.stream, m, k, _addr(x), _addr(norm_w), _addr(out)))

    def q4_gemm(self, m, k, n, x, codes, gscales, y=None, y_bf16=None, residual=None, x_dtype=QM_F16):
        """y (f32) or y_bf16 [m, n] = x (f16 or bf16 [m, k]) @ W (+ residual)."""
        self._check(self.lib.qm_q4_gemm(self.h, self.stream, m, k, n, _addr(x), x_dtype, _addr(codes),
                                        _addr(gscales), _addr(residual), _addr(y), _addr(y_bf16)))

    def q4_gemm_gate_up(self, m, k, n, x, gate_codes, gate_gscales, up_codes, up_gscales, out_bf16,
                        x_dtype=QM_F16):
        """out_bf16 [m, n] = bf16(silu(x @ Wg) * (x @ Wu)), x f16 or bf16 [m, k]."""
        self._check(self.lib.qm_q4_gemm_gate_up(self.h, self.stream, m, k, n, _addr(x), x_dtype,
                                                _addr(gate_codes), _addr(gate_gscales), _addr(up_codes),
                                                _addr(up_gscales), _addr(out_bf16)))

    def q4_gate_up(self, k, n, x, norm_w, gate_codes, gate_gscales, up_codes, up_gscales, out):
        """out[n] = silu(xn @ Wg) * (xn @ Wu), xn = rms_norm(x, norm_w) or x."""
        self._check(self.lib.qm_q4_gate_up(self.h, self.stream, k, n, _addr(x), _addr(norm_w),
                                           _addr(gate_codes), _addr(gate_gscales), _addr(up_codes),
                                           _addr(up_gscales), _addr(out)))


    def q4_lm_head(self, vocab, hidden, x, norm_w, packed, scales, logits):
        """logits [vocab] = (rms_norm(x, norm_w) or x) . each row of the Q4 embedding."""
        self._check(self.lib.qm_q4_lm_head(self.h, self.stream, vocab, hidden, _addr(x), _addr(norm_w),
                                           _addr(packed), _addr(scales), _addr(logits)))

    def q4_embed(self, count, vocab, hidden, ids, packed, scales, out):
        """out [count, hidden] = the dequantized embedding rows of ids (int32 [count])."""
        self._check(self.lib.qm_q4_embed(self.h, self.stream, count, vocab, hidden, _addr(ids), _addr(packed),
                                         _addr(scales), _addr(out)))


    def sample(self, vocab, logits, generated, n_generated, rng_state, token_out, temperature=1.0, top_p=0.95,
               top_k=20, repetition_penalty=1.0, presence_penalty=0.0, banned_id=-1, flags=0,
               top_ids=None, top_probs=None):
        """Penalties (in place on logits) and the next token into token_out (int32 [1]);
        rng_state is the device uint64 xorshift64 state."""
        p = QmSampleParams(temperature, top_p, top_k, repetition_penalty, presence_penalty, banned_id, flags)
        self._check(self.lib.qm_sample(self.h, self.stream, vocab, _addr(logits), _addr(generated), n_generated,
                                       C.byref(p), _addr(rng_state), _addr(token_out), _addr(top_ids),
                                       _addr(top_probs)))


class Event:
    def __init__(self, ctx: Context):
        self.ctx = ctx
        e = _P(0)
        ctx._check(ctx.lib.qm_event_create(ctx.h, C.byref(e)))
        self.h = e.value

    def record(self):
        self.ctx._check(self.ctx.lib.qm_event_record(self.ctx.h, self.h, self.ctx.stream))

    def elapsed_ms(self, later: "Event") -> float:
        ms = C.c_float(0)
        self.ctx._check(self.ctx.lib.qm_event_elapsed_ms(self.ctx.h, self.h, later.h, C.byref(ms)))
        return float(ms.value)

    def __del__(self):
        try:
            if self.h and self.ctx.h:
                self.ctx.lib.qm_event_destroy(self.ctx.h, self.h)
        except Exception:
            pass


class Graph:
    def __init__(self, ctx: Context, h: int):
        self.ctx = ctx
        self.h = h

    def launch(self):
        self.ctx._check(self.ctx.lib.qm_graph_launch(self.ctx.h, self.h, self.ctx.stream))

    def close(self):
        if self.h and self.ctx.h:
            self.ctx.lib.qm_graph_destroy(self.ctx.h, self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
