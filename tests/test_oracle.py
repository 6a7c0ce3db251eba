"""Pins for the CPU oracle (oracle/qora_oracle.c).

The reference ships no tests, fixtures or golden vectors, and its Rust
toolchain is not available, so every oracle function is pinned here by what
the mathematics fixes: closed forms, invariants, brute force on tiny inputs
and float64 shadows written in a different form from the oracle's loops
(matrix / paper form).  Each check is chosen so that a plausible slip (a
dropped term, a transposed state, a wrong head map, (1+g) vs g, a missing
scale) fails it.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import load_oracle

O = load_oracle()
RNG = np.random.default_rng(1234)


def f64(x):
    return np.asarray(x, np.float64)


# ---------------------------------------------------------------- conversions
def test_f16_conversion_matches_ieee():
    vals = np.concatenate([
        RNG.standard_normal(2000).astype(np.float32) * 10,
        np.array([0.0, -0.0, 1.0, -2.5, 65504.0, 65519.0, 65520.0, 1e-8, 6.0e-8, 5.96e-8,
                  3e-5, 6.1e-5, 6.104e-5, np.inf, -np.inf], np.float32),
        (RNG.standard_normal(500) * 1e-6).astype(np.float32),
    ])
    got = O.f16_bits(vals)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    allbits = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    finite = ~np.isnan(allbits.view(np.float16))
    back = O.f16_to_f32(allbits[finite])
    assert np.array_equal(back, allbits[finite].view(np.float16).astype(np.float32))


def test_bf16_round_to_nearest_even():
    lib = O.lib()
    vals = np.concatenate([RNG.standard_normal(3000) * 100, [2.0 ** -130, 3.0e38, -1e-3]]).astype(np.float32)
    for v in vals:
        b = lib.or_f32_to_bf16(float(v))
        got = lib.or_bf16_to_f32(b)
        # the two bf16 neighbours of v: truncation and one step away from zero
        lo = np.uint32(v.view(np.uint32) & 0xFFFF0000).view(np.float32)
        hi = np.uint32((v.view(np.uint32) & 0xFFFF0000) + 0x10000).view(np.float32)
        assert got in (lo, hi)
        assert abs(f64(got) - f64(v)) <= abs(f64(lo if got == hi else hi) - f64(v))
    # ties go to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7
    assert lib.or_f32_to_bf16(1.0 + 2 ** -8) == 0x3F80
    assert lib.or_f32_to_bf16(1.0 + 3 * 2 ** -8) == 0x3F82
    assert lib.or_bf16_to_f32(0x3F82) == np.float32(1.015625)


# ---------------------------------------------------------------- scalars
def test_silu_softplus_closed_forms():
    assert O.silu(0.0) == 0.0
    assert abs(O.silu(1.0) - 1.0 / (1.0 + np.exp(-1.0))) < 1e-7
    assert abs(O.silu(-3.0) - (-3.0 / (1.0 + np.exp(3.0)))) < 1e-7
    # softplus: identity strictly above 20, log1p(exp) at and below it
    assert O.softplus(25.0) == 25.0
    assert O.softplus(20.5) == 20.5
    assert abs(O.softplus(20.0) - np.log1p(np.exp(20.0))) < 1e-5
    assert abs(O.softplus(0.0) - np.log(2.0)) < 1e-7
    assert abs(O.softplus(-5.0) - np.log1p(np.exp(-5.0))) < 1e-8


def test_l2_normalize():
    x = RNG.standard_normal(128).astype(np.float32)
    y = O.l2_normalize(x)
    assert abs(np.linalg.norm(f64(y)) - 1.0) < 1e-6
    assert np.allclose(y, x / np.linalg.norm(f64(x)), rtol=1e-6, atol=0)
    assert np.array_equal(O.l2_normalize(np.zeros(16, np.float32)), np.zeros(16, np.float32))
    tiny = np.full(4, 1e-14, np.float32)          # norm 2e-14 <= 1e-12: untouched
    assert np.array_equal(O.l2_normalize(tiny), tiny)


def test_softmax_raw():
    x = (RNG.standard_normal(300) * 4).astype(np.float32)
    p = O.softmax_raw(x)
    e = np.exp(f64(x) - f64(x).max())
    assert abs(p.sum() - 1.0) < 1e-5
    assert np.allclose(p, e / e.sum(), rtol=1e-5, atol=1e-9)
    assert np.allclose(O.softmax_raw(x + 7.0), p, rtol=1e-5, atol=1e-9)


def test_rms_norm_one_plus_gamma():
    x = RNG.standard_normal(2560).astype(np.float32)
    g = (0.1 * RNG.standard_normal(2560)).astype(np.float16)
    out = O.rms_norm(x, g.view(np.uint16))
    ref = f64(x) / np.sqrt(np.mean(f64(x) ** 2) + 1e-6) * (1.0 + f64(g))
    assert np.allclose(out, ref, rtol=2e-6, atol=1e-7)
    # a constant vector c normalises to c / sqrt(c^2 + eps) * (1 + g)
    c = np.full(64, 3.0, np.float32)
    g0 = np.zeros(64, np.uint16)
    assert np.allclose(O.rms_norm(c, g0), 3.0 / np.sqrt(9.0 + 1e-6), rtol=1e-7)


def test_per_head_rms_norm_heads_independent():
    x = RNG.standard_normal((4, 256)).astype(np.float32)
    x[2] *= 100.0
    g = (0.1 * RNG.standard_normal(256)).astype(np.float16)
    out = O.per_head_rms_norm(x.ravel(), 4, 256, g.view(np.uint16)).reshape(4, 256)
    for h in range(4):
        ref = f64(x[h]) / np.sqrt(np.mean(f64(x[h]) ** 2) + 1e-6) * (1.0 + f64(g))
        assert np.allclose(out[h], ref, rtol=2e-6, atol=1e-7)


# ---------------------------------------------------------------- RoPE
def test_rope_table_formula():
    cos, sin = O.rope_table(8192)
    assert cos.shape == (8192, 32)
    assert np.array_equal(cos[0], np.ones(32, np.float32)) and np.array_equal(sin[0], np.zeros(32, np.float32))
    # freq_i = theta^(-2i/64); f32 rounding of freq and angle bounds the error
    pos = np.array([1, 2, 17, 1000, 4096, 8191])
    freq = 1.0 / (1e7 ** (2.0 * np.arange(32) / 64.0))
    ang = pos[:, None] * freq[None, :]
    tol = 1e-6 + 4 * np.abs(ang) * 2 ** -23
    assert np.all(np.abs(f64(cos[pos]) - np.cos(ang)) <= tol)
    assert np.all(np.abs(f64(sin[pos]) - np.sin(ang)) <= tol)
    # the lowest frequency rotates slowest: freq_31 ~ 1e7^(-31/32)
    assert abs(np.arccos(np.clip(cos[1, 0], -1, 1)) - 1.0) < 1e-6


def test_partial_rope_invariants():
    H, D = 4, 256
    cos, sin = O.rope_table(64)
    x = RNG.standard_normal(H * D).astype(np.float32)
    assert np.array_equal(O.apply_partial_rope(x, H, D, cos, sin, 64, 0), x)   # pos 0: identity
    y = O.apply_partial_rope(x, H, D, cos, sin, 64, 37).reshape(H, D)
    xr = x.reshape(H, D)
    assert np.array_equal(y[:, 64:], xr[:, 64:])                               # dims >= 64 untouched
    # pairs (i, i+32) rotate by the angle of row 37: explicit 2x2 rotation in f64
    c, s = f64(cos[37]), f64(sin[37])
    x1, x2 = f64(xr[:, :32]), f64(xr[:, 32:64])
    assert np.allclose(y[:, :32], x1 * c - x2 * s, atol=1e-6)
    assert np.allclose(y[:, 32:64], x2 * c + x1 * s, atol=1e-6)
    assert np.allclose(np.hypot(y[:, :32], y[:, 32:64]), np.hypot(x1, x2), rtol=1e-6)
    # relative position: <R_m q, R_n k> depends only on m - n
    q = RNG.standard_normal(D).astype(np.float32)
    k = RNG.standard_normal(D).astype(np.float32)
    d1 = np.dot(f64(O.apply_partial_rope(q, 1, D, cos, sin, 64, 20)), f64(O.apply_partial_rope(k, 1, D, cos, sin, 64, 5)))
    d2 = np.dot(f64(O.apply_partial_rope(q, 1, D, cos, sin, 64, 40)), f64(O.apply_partial_rope(k, 1, D, cos, sin, 64, 25)))
    assert abs(d1 - d2) < 1e-4


# ---------------------------------------------------------------- conv1d
def test_conv1d_impulse_and_padding():
    n, ks = 8, 4
    w = RNG.standard_normal((n, ks)).astype(np.float32)
    buf = np.zeros((n, ks - 1), np.float32)
    outs = []
    for t in range(6):
        x = np.ones(n, np.float32) if t == 0 else np.zeros(n, np.float32)
        outs.append(O.conv1d_step(buf, w, x))
    outs = np.array(outs)
    # impulse at t=0 comes back as the taps newest-first: w[:,3], w[:,2], w[:,1], w[:,0], 0
    for t in range(4):
        assert np.array_equal(outs[t], w[:, 3 - t])
    assert np.array_equal(outs[4], np.zeros(n, np.float32))
    # general input vs direct causal convolution with zero history
    buf = np.zeros((n, ks - 1), np.float32)
    xs = RNG.standard_normal((10, n)).astype(np.float32)
    got = np.array([O.conv1d_step(buf, w, xs[t]) for t in range(10)])
    xp = np.vstack([np.zeros((ks - 1, n)), f64(xs)])
    ref = np.array([(xp[t:t + ks] * f64(w).T).sum(0) for t in range(10)])
    assert np.allclose(got, ref, atol=1e-5)
    assert np.array_equal(buf, xs[-3:].T)        # buffer holds the last 3 raw inputs, oldest first


# ---------------------------------------------------------------- delta rule
def _delta_rule_paper(S, q, k, v, alpha, beta):
    """Gated delta rule in the paper's form: S' = alpha S (I - beta k k^T) + beta v k^T, y = S' q."""
    S, q, k, v = f64(S), f64(q), f64(k), f64(v)
    n = k.size
    Sn = alpha * S @ (np.eye(n) - beta * np.outer(k, k)) + beta * np.outer(v, k)
    return Sn, Sn @ q


@pytest.mark.parametrize("kind", [O.UPDATE_SCALAR, O.UPDATE_AVX512_EMUL])
def test_head_update_vs_paper_form(kind):
    hd = 128
    S = (0.02 * RNG.standard_normal((hd, hd))).astype(np.float32)
    q = O.l2_normalize(RNG.standard_normal(hd).astype(np.float32)) / np.sqrt(np.float32(hd))
    k = O.l2_normalize(RNG.standard_normal(hd).astype(np.float32))
    v = RNG.standard_normal(hd).astype(np.float32)
    Sn, y = O.head_update(S.ravel(), q, k, v, 0.93, 0.6, kind)
    Sr, yr = _delta_rule_paper(S, q, k, v, 0.93, 0.6)
    assert np.abs(Sn.reshape(hd, hd) - Sr).max() < 1e-5
    assert np.abs(y - yr).max() < 1e-5


def test_head_update_special_cases():
    hd = 32
    S = RNG.standard_normal((hd, hd)).astype(np.float32)
    q = RNG.standard_normal(hd).astype(np.float32)
    k = O.l2_normalize(RNG.standard_normal(hd).astype(np.float32))
    v = RNG.standard_normal(hd).astype(np.float32)
    # alpha = beta = 1, |k| = 1: the delta rule stores v at key k exactly
    Sn, _ = O.head_update(S.ravel(), q, k, v, 1.0, 1.0)
    assert np.abs(f64(Sn.reshape(hd, hd)) @ f64(k) - f64(v)).max() < 1e-4
    # beta = 0: pure decay, y = alpha S q
    Sn, y = O.head_update(S.ravel(), q, k, v, 0.5, 0.0)
    assert np.array_equal(Sn, (S * np.float32(0.5)).ravel())
    assert np.allclose(y, 0.5 * f64(S) @ f64(q), atol=1e-5)
    # alpha = 0: S' = beta v k^T, y = beta (k.q) v
    Sn, y = O.head_update(S.ravel(), q, k, v, 0.0, 0.7)
    assert np.allclose(Sn.reshape(hd, hd), 0.7 * np.outer(f64(v), f64(k)), atol=1e-6)
    assert np.allclose(y, 0.7 * np.dot(f64(k), f64(q)) * f64(v), atol=1e-5)
    # rows are independent: perturbing row 5 of S changes only row 5 / y[5]
    S2 = S.copy()
    S2[5] += 1.0
    A, ya = O.head_update(S.ravel(), q, k, v, 0.9, 0.4)
    B, yb = O.head_update(S2.ravel(), q, k, v, 0.9, 0.4)
    diff = np.any(A.reshape(hd, hd) != B.reshape(hd, hd), axis=1)
    assert diff[5] and diff.sum() == 1
    assert np.flatnonzero(ya != yb).tolist() == [5]


def test_avx512_intrinsics_match_lane_emulation():
    if not O.has_avx512():
        pytest.skip("host has no AVX-512F")
    hd = 128
    for seed in range(3):
        r = np.random.default_rng(seed)
        S = (0.02 * r.standard_normal(hd * hd)).astype(np.float32)
        q, k, v = (r.standard_normal((3, hd)).astype(np.float32))
        a = O.head_update(S, q, k, v, 0.97, 0.55, O.UPDATE_AVX512)
        b = O.head_update(S, q, k, v, 0.97, 0.55, O.UPDATE_AVX512_EMUL)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
        c = O.head_update(S, q, k, v, 0.97, 0.55, O.UPDATE_SCALAR)
        assert np.abs(a[1] - c[1]).max() < 1e-5 * max(1.0, np.abs(c[1]).max())


# ---------------------------------------------------------------- DeltaNet layer slices
def _tiny_cfg():
    return O.config(num_qk_heads=2, num_v_heads=4, dn_head_dim=16, conv_kernel=4)


def _dn_inputs(cfg, T, seed):
    r = np.random.default_rng(seed)
    hd, nv, nqk = cfg.dn_head_dim, cfg.num_v_heads, cfg.num_qk_heads
    qkv_dim = (2 * nqk + nv) * hd
    return dict(
        qkv=r.standard_normal((T, qkv_dim)).astype(np.float32),
        a=r.standard_normal((T, nv)).astype(np.float32),
        b=r.standard_normal((T, nv)).astype(np.float32),
        z=r.standard_normal((T, nv * hd)).astype(np.float32),
        conv_w=(0.5 * r.standard_normal((qkv_dim, 4))).astype(np.float32),
        a_log=np.log(r.uniform(0.01, 0.1, nv)).astype(np.float32),
        dt_bias=(0.1 * r.standard_normal(nv)).astype(np.float32),
        norm_w=(1 + 0.1 * r.standard_normal(hd)).astype(np.float16).view(np.uint16),
        S0=(0.02 * r.standard_normal((nv, hd, hd))).astype(np.float32),
    )


def _dn_token_f64(cfg, act, a, b, z, a_log, dt_bias, norm_w, S):
    """One token from the definitions, float64, matrix form."""
    hd, nv, nqk = cfg.dn_head_dim, cfg.num_v_heads, cfg.num_qk_heads
    act = f64(act)
    q = act[:nqk * hd].reshape(nqk, hd)
    k = act[nqk * hd:2 * nqk * hd].reshape(nqk, hd)
    v = act[2 * nqk * hd:].reshape(nv, hd)
    q = q / np.linalg.norm(q, axis=1, keepdims=True) / np.sqrt(hd)
    k = k / np.linalg.norm(k, axis=1, keepdims=True)
    sp = np.log1p(np.exp(f64(a) + f64(dt_bias)))
    alpha = np.exp(-np.exp(f64(a_log)) * sp)
    beta = 1.0 / (1.0 + np.exp(-f64(b)))
    g = f64(norm_w.view(np.float16))
    out = np.empty((nv, hd))
    for vh in range(nv):
        j = vh * nqk // nv                       # consecutive GVA map
        S[vh], y = _delta_rule_paper(S[vh], q[j], k[j], v[vh], alpha[vh], beta[vh])
        yn = y / np.sqrt(np.mean(y ** 2) + 1e-6) * g
        zz = f64(z).reshape(nv, hd)[vh]
        out[vh] = yn * zz / (1.0 + np.exp(-zz))
    return out.ravel()


@pytest.mark.parametrize("kind", [O.UPDATE_SCALAR, O.UPDATE_AVX512_EMUL])
def test_deltanet_decode_step_vs_definitions(kind):
    cfg = _tiny_cfg()
    d = _dn_inputs(cfg, 8, 7)
    S = d["S0"].copy()
    S64 = f64(d["S0"]).copy()
    buf = np.zeros((d["qkv"].shape[1], 3), np.float32)
    xs_hist = np.zeros((3, d["qkv"].shape[1]))
    for t in range(8):
        out = O.deltanet_decode_step(cfg, d["qkv"][t], d["a"][t], d["b"][t], d["z"][t], d["conv_w"],
                                     d["a_log"], d["dt_bias"], d["norm_w"], S, buf, preact=True,
                                     kind=kind)
        window = np.vstack([xs_hist, f64(d["qkv"][t])[None]])
        conv = (window * f64(d["conv_w"]).T).sum(0)
        xs_hist = window[1:]
        act = conv / (1.0 + np.exp(-conv))
        ref = _dn_token_f64(cfg, act, d["a"][t], d["b"][t], d["z"][t], d["a_log"], d["dt_bias"],
                            d["norm_w"], S64)
        assert np.abs(out - ref).max() < 2e-5, t
    assert np.abs(S - S64).max() < 1e-5


def test_deltanet_decode_gva_map_is_consecutive():
    """v heads 2j and 2j+1 read q/k head j (gemv.rs:806), not j and j+H/2."""
    cfg = _tiny_cfg()
    d = _dn_inputs(cfg, 1, 3)
    hd = cfg.dn_head_dim
    S = np.zeros((cfg.num_v_heads, hd, hd), np.float32)
    qkv = d["qkv"][0].copy()
    qkv[hd:2 * hd] = 0.0          # q head 1 zero -> y = 0 for v heads 2, 3 only
    out = O.deltanet_decode_step(cfg, qkv, d["a"][0], d["b"][0], d["z"][0], d["conv_w"],
                                 d["a_log"], d["dt_bias"], d["norm_w"], S)
    o = out.reshape(cfg.num_v_heads, hd)
    assert np.all(o[2:] == 0.0) and np.all(np.abs(o[:2]).sum(1) > 0)


def test_deltanet_decode_heads_parallel_equals_serial():
    """The v-head loop split over threads (the CPU baseline's all-cores
    variant) gives the serial loop's state and output bit for bit, at the
    full dimensions with a conv step."""
    cfg = O.config()
    rng = np.random.default_rng(77)
    qkv = rng.standard_normal(8192).astype(np.float32)
    a, b = rng.standard_normal(32).astype(np.float32), rng.standard_normal(32).astype(np.float32)
    z = rng.standard_normal(4096).astype(np.float32)
    conv_w = (0.5 * rng.standard_normal((8192, 4))).astype(np.float32)
    a_log = np.log(rng.uniform(0.01, 0.1, 32)).astype(np.float32)
    dt_bias = np.zeros(32, np.float32)
    nw = O.f16_bits(1.0 + 0.1 * rng.standard_normal(128))
    S0 = (0.02 * rng.standard_normal((32, 128, 128))).astype(np.float32)
    buf0 = rng.standard_normal((8192, 3)).astype(np.float32)
    res = []
    for nt in (1, 4):
        S, buf = S0.copy(), buf0.copy()
        out = O.deltanet_decode_step(cfg, qkv, a, b, z, conv_w, a_log, dt_bias, nw, S,
                                     conv_buf=buf, preact=True, nthreads=nt)
        res.append((out, S, buf))
    for x, y in zip(res[0], res[1]):
        assert np.array_equal(x, y)


def test_deltanet_prefill_equals_decode_steps():
    """The sequential prefill (gemv.rs:1119-1219) is T scalar decode steps, bit for bit."""
    cfg = _tiny_cfg()
    T = 12
    d = _dn_inputs(cfg, T, 11)
    S1, S2 = d["S0"].copy(), d["S0"].copy()
    b1 = (0.3 * np.random.default_rng(1).standard_normal((d["qkv"].shape[1], 3))).astype(np.float32)
    b2 = b1.copy()
    outp = O.deltanet_prefill(cfg, d["qkv"], d["a"], d["b"], d["z"], d["conv_w"], d["a_log"],
                              d["dt_bias"], d["norm_w"], S1, b1)
    for t in range(T):
        o = O.deltanet_decode_step(cfg, d["qkv"][t], d["a"][t], d["b"][t], d["z"][t], d["conv_w"],
                                   d["a_log"], d["dt_bias"], d["norm_w"], S2, b2, preact=True,
                                   kind=O.UPDATE_SCALAR)
        assert np.array_equal(o, outp[t])
    assert np.array_equal(S1, S2) and np.array_equal(b1, b2)


# ---------------------------------------------------------------- attention
def _attn_cfg():
    return O.config(num_heads=4, num_kv_heads=2, attn_head_dim=32, rope_dim=16)


def _attention_f64(q, K, V, groups):
    """Textbook softmax(q K^T / sqrt(D)) V per head, kv head h // groups."""
    H, D = q.shape
    out = np.empty((H, D))
    for h in range(H):
        s = f64(K[:, h // groups]) @ f64(q[h]) / np.sqrt(D)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ f64(V[:, h // groups])
    return out


def test_attn_decode_vs_textbook():
    cfg = _attn_cfg()
    H, KV, D = 4, 2, 32
    r = np.random.default_rng(5)
    L = 40
    cos, sin = O.rope_table(64, rope_dim=16)
    qg = r.standard_normal((H, 2 * D)).astype(np.float32)
    kn, vn = r.standard_normal((2, KV, D)).astype(np.float32)
    qn = (0.1 * r.standard_normal(D)).astype(np.float16).view(np.uint16)
    knw = (0.1 * r.standard_normal(D)).astype(np.float16).view(np.uint16)
    Kc = np.zeros((L + 1, KV, D), np.float32)
    Vc = np.zeros((L + 1, KV, D), np.float32)
    Kc[:L], Vc[:L] = r.standard_normal((2, L, KV, D)).astype(np.float32)
    out = O.attn_decode_step(cfg, qg, kn, vn, qn, knw, cos, sin, Kc, Vc, L)
    # expected: q/k normed with (1+g), roped at position L, appended, attended, gated
    q = O.apply_partial_rope(O.per_head_rms_norm(qg.reshape(H, 2, D)[:, 0].ravel(), H, D, qn), H, D, cos, sin, 16, L)
    k = O.apply_partial_rope(O.per_head_rms_norm(kn.ravel(), KV, D, knw), KV, D, cos, sin, 16, L)
    assert np.array_equal(Kc[L], k.reshape(KV, D)) and np.array_equal(Vc[L], vn)
    att = _attention_f64(q.reshape(H, D), Kc, Vc, H // KV)
    gate = f64(qg.reshape(H, 2, D)[:, 1])
    ref = att / (1.0 + np.exp(-gate))
    assert np.abs(out.reshape(H, D) - ref).max() < 1e-5


def test_attn_decode_limits_and_threads():
    cfg = _attn_cfg()
    H, KV, D = 4, 2, 32
    r = np.random.default_rng(9)
    cos, sin = O.rope_table(128, rope_dim=16)
    qg = r.standard_normal((H, 2 * D)).astype(np.float32)
    kn, vn = r.standard_normal((2, KV, D)).astype(np.float32)
    z16 = np.zeros(D, np.uint16)
    # L = 1 (empty cache): softmax over one key -> out = v_new[h//2] * sigmoid(gate)
    Kc = np.zeros((1, KV, D), np.float32)
    Vc = np.zeros((1, KV, D), np.float32)
    out = O.attn_decode_step(cfg, qg, kn, vn, z16, z16, cos, sin, Kc, Vc, 0).reshape(H, D)
    gate = f64(qg.reshape(H, 2, D)[:, 1])
    for h in range(H):
        assert np.allclose(out[h], f64(vn[h // 2]) / (1 + np.exp(-gate[h])), atol=1e-6)
    # identical keys -> uniform weights -> mean of V
    L = 70
    Kc = np.zeros((L + 1, KV, D), np.float32)
    Vc = r.standard_normal((L + 1, KV, D)).astype(np.float32)
    Kc[:] = 0.0
    kz = np.zeros((KV, D), np.float32)        # new key normalises to 0 as well
    out = O.attn_decode_step(cfg, qg, kz, Vc[L].copy(), z16, z16, cos, sin, Kc, Vc, L).reshape(H, D)
    for h in range(H):
        assert np.allclose(out[h], f64(Vc[:, h // 2]).mean(0) / (1 + np.exp(-gate[h])), atol=1e-5)
    # thread count does not change per-head arithmetic (rayon split, gemv.rs:963)
    Kc = r.standard_normal((L + 1, KV, D)).astype(np.float32)
    Vc = r.standard_normal((L + 1, KV, D)).astype(np.float32)
    K2, V2 = Kc.copy(), Vc.copy()
    o1 = O.attn_decode_step(cfg, qg, kn, vn, z16, z16, cos, sin, Kc, Vc, L, nthreads=1)
    o4 = O.attn_decode_step(cfg, qg, kn, vn, z16, z16, cos, sin, K2, V2, L, nthreads=4)
    assert np.array_equal(o1, o4)
    with pytest.raises(IndexError):
        O.attn_decode_step(cfg, qg, kn, vn, z16, z16, cos, sin, np.zeros((200, KV, D), np.float32),
                           np.zeros((200, KV, D), np.float32), 128)


def test_attn_prefill_vs_decode_and_textbook():
    cfg = _attn_cfg()
    H, KV, D = 4, 2, 32
    S = 24
    r = np.random.default_rng(13)
    cos, sin = O.rope_table(64, rope_dim=16)
    qg = r.standard_normal((S, H, 2 * D)).astype(np.float32)
    k = r.standard_normal((S, KV, D)).astype(np.float32)
    v = r.standard_normal((S, KV, D)).astype(np.float32)
    qn = (0.1 * r.standard_normal(D)).astype(np.float16).view(np.uint16)
    kn = (0.1 * r.standard_normal(D)).astype(np.float16).view(np.uint16)
    out, Kc, Vc = O.attn_prefill(cfg, qg, k, v, qn, kn, cos, sin, nthreads=2)
    out = out.reshape(S, H, D)
    assert np.array_equal(Vc, v)
    gate = f64(qg[:, :, D:])
    # row 0 attends only to itself: v_0 * sigmoid(gate)
    for h in range(H):
        assert np.allclose(out[0, h], f64(v[0, h // 2]) / (1 + np.exp(-gate[0, h])), atol=1e-6)
    # every row t equals a decode step at seq_len = t over the prefilled cache
    for t in [1, 7, S - 1]:
        Kd = np.zeros((t + 1, KV, D), np.float32)
        Vd = np.zeros((t + 1, KV, D), np.float32)
        Kd[:t], Vd[:t] = Kc[:t], Vc[:t]
        od = O.attn_decode_step(cfg, qg[t].ravel(), k[t], v[t], qn, kn, cos, sin, Kd, Vd, t)
        assert np.array_equal(Kd[t], Kc[t])
        assert np.array_equal(od.reshape(H, D), out[t])
    # causal textbook attention in f64
    for t in [3, S - 1]:
        q = O.apply_partial_rope(O.per_head_rms_norm(qg[t, :, :D].ravel(), H, D, qn), H, D, cos, sin, 16, t)
        ref = _attention_f64(q.reshape(H, D), Kc[:t + 1], Vc[:t + 1], 2) / (1 + np.exp(-gate[t]))
        assert np.abs(out[t] - ref).max() < 1e-5
    # a row subset reproduces the same rows
    sub, _, _ = O.attn_prefill(cfg, qg, k, v, qn, kn, cos, sin, rows=[5, 17])
    sub = sub.reshape(S, H, D)
    assert np.array_equal(sub[5], out[5]) and np.array_equal(sub[17], out[17])
    assert np.all(sub[6] == 0)
