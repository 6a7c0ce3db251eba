"""GPU parity: Q4 projections (qm_q4_repack, qm_q4_gemv) vs the CPU oracle.

The weight goes to the device in the reference layout and is repacked
there; the repack must equal the numpy tile-major transposition exactly.
The oracle restates gemv_q4_inner (gemv.rs:412-445) with the reference's
k-ordered fp32 sums; the kernel sums in another fixed order.  Bar: per
output column |y - y_ref| <= 1e-5 * sum_k |x_k W_kj| (fp32 reassociation
over up to 12000 terms), and bit-identical results run to run.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import load_mixer, load_oracle, load_workloads

pytestmark = pytest.mark.gpu

M = load_mixer()
O = load_oracle()
W = load_workloads()


def repack(ctx, packed, scales):
    k, n = packed.shape[0], packed.shape[1] * 2
    dp, ds = ctx.upload(packed), ctx.upload(scales)
    codes, gsc = ctx.alloc(k * n // 2), ctx.alloc(max(16, k * (n // 32) * 2))
    ctx.q4_repack(k, n, dp, ds, codes, gsc)
    return codes, gsc


def run_gpu(ctx, x, packed, scales):
    k, n = packed.shape[0], packed.shape[1] * 2
    codes, gsc = repack(ctx, packed, scales)
    dx, y = ctx.upload(x), ctx.alloc(n * 4)
    ctx.q4_gemv(k, n, dx, codes, gsc, y)
    return ctx.download(y, (n,), np.float32)


def check(got, x, packed, scales):
    ref = O.q4_gemv(x, packed, scales)
    mag = np.abs(x).astype(np.float64) @ np.abs(W.q4_dequant(packed, scales)).astype(np.float64)
    err = np.abs(got.astype(np.float64) - ref)
    print(f"max|d| {err.max():.3e}  max|d|/mag {(err / (mag + 1e-30)).max():.3e}")
    assert np.all(err <= 1e-5 * mag + 1e-30)


@pytest.mark.parametrize("name", ["in_proj_qkv", "in_proj_a", "in_proj_z", "out_proj", "k_proj", "down_proj"])
def test_q4_gemv_projection_shapes(ctx, name):
    k, n = W.Q4_PROJ_SHAPES[name]
    w = W.q4_gemv_workload(k, n, seed=k + n)
    w["x"][::5] = 0.0
    print(f"case: q4 gemv {name} k={k} n={n}", flush=True)
    got = run_gpu(ctx, w["x"], w["packed"], w["scales"])
    check(got, w["x"], w["packed"], w["scales"])
    again = run_gpu(ctx, w["x"], w["packed"], w["scales"])
    assert np.array_equal(got, again)


@pytest.mark.parametrize("k,n", [(1, 32), (37, 64), (513, 96), (1000, 2592), (4096, 32), (4097, 288),
                                 (12000, 64)])
def test_q4_gemv_ragged(ctx, k, n):
    w = W.q4_gemv_workload(k, n, seed=k)
    print(f"case: q4 gemv ragged k={k} n={n}", flush=True)
    check(run_gpu(ctx, w["x"], w["packed"], w["scales"]), w["x"], w["packed"], w["scales"])


def test_q4_gemv_multi_layer_projections(ctx):
    """in_proj_qkv, in_proj_z, in_proj_a, in_proj_b of one input in one launch,
    each output as its own qm_q4_gemv would give it (bit for bit) and within
    the bar of the oracle."""
    rng = np.random.default_rng(21)
    x = rng.standard_normal(2560).astype(np.float32)
    names = ["in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b"]
    ws = [W.q4_random_weight(*W.Q4_PROJ_SHAPES[nm], rng) for nm in names]
    dev = [repack(ctx, p, s) for p, s in ws]
    ns = [W.Q4_PROJ_SHAPES[nm][1] for nm in names]
    ys = [ctx.alloc(n * 4) for n in ns]
    dx = ctx.upload(x)
    print("case: q4 gemv multi (qkv, z, a, b)", flush=True)
    ctx.q4_gemv_multi(2560, dx, [(n, c, g, y) for n, (c, g), y in zip(ns, dev, ys)])
    for (p, s), n, (c, g), y in zip(ws, ns, dev, ys):
        got = ctx.download(y, (n,), np.float32)
        check(got, x, p, s)
        single = ctx.alloc(n * 4)
        ctx.q4_gemv(2560, n, dx, c, g, single)
        assert np.array_equal(got, ctx.download(single, (n,), np.float32))
    with pytest.raises(M.MixerError) as e:
        ctx.q4_gemv_multi(2560, dx, [(ns[0], dev[0][0], dev[0][1], ys[0])] * 5)
    assert e.value.code == 3


@pytest.mark.parametrize("k,n", [(2560, 8192), (37, 96), (1, 32), (130, 544), (70, 4096)])
def test_q4_repack_is_the_tile_major_transpose(ctx, k, n):
    rng = np.random.default_rng(k + n)
    packed, scales = W.q4_random_weight(k, n, rng)
    print(f"case: q4 repack k={k} n={n}", flush=True)
    codes, gsc = repack(ctx, packed, scales)
    want_c, want_s = W.q4_device_layout(packed, scales)
    assert np.array_equal(ctx.download(codes, want_c.shape, np.uint8), want_c)
    assert np.array_equal(ctx.download(gsc, want_s.shape, np.uint16), want_s)


def test_q4_gemv_quantized_weight(ctx):
    """A weight quantized by the oracle's quantize_q4 (not random codes)."""
    rng = np.random.default_rng(9)
    wf = (0.02 * rng.standard_normal((2560, 1024))).astype(np.float32)
    packed, scales = O.q4_quantize(wf)
    x = rng.standard_normal(2560).astype(np.float32)
    print("case: q4 gemv quantized weight", flush=True)
    check(run_gpu(ctx, x, packed, scales), x, packed, scales)


def test_q4_gemv_errors(ctx):
    w = W.q4_gemv_workload(64, 64, seed=1)
    dx, y = ctx.upload(w["x"]), ctx.alloc(64 * 4)
    dp, ds = repack(ctx, w["packed"], w["scales"])
    with pytest.raises(M.MixerError) as e:
        ctx.q4_gemv(64, 48, dx, dp, ds, y)           # n not a multiple of 32
    assert e.value.code == 4
    with pytest.raises(M.MixerError) as e:
        ctx.q4_gemv(64, 64, dx.offset(4), dp, ds, y)  # misaligned x
    assert e.value.code == 3
    with pytest.raises(M.MixerError) as e:
        ctx.q4_gemv(0, 64, dx, dp, ds, y)
    assert e.value.code == 3
    with pytest.raises(M.MixerError) as e:
        ctx.q4_repack(64, 40, dp, ds, dp, ds)        # n not a multiple of 32
    assert e.value.code == 4


def _mag(x, packed, scales):
    return np.abs(x).astype(np.float64) @ np.abs(W.q4_dequant(packed, scales)).astype(np.float64)


def test_q4_gemv_multi_norm_and_residual(ctx):
    """rms_norm(x, 1 + gamma) fused ahead of three projections, and a
    residual add (in place, y = residual) on one of them (gemv.rs:571-579,
    :889-890)."""
    rng = np.random.default_rng(31)
    k = 2560
    x = (3.0 * rng.standard_normal(k)).astype(np.float32)
    gamma = W.f16_bits(0.1 * rng.standard_normal(k).astype(np.float32))
    xn = O.rms_norm(x, gamma)
    shapes = [(k, 1024), (k, 8192), (k, 32)]
    ws = [W.q4_random_weight(kk, n, rng) for kk, n in shapes]
    dev = [repack(ctx, p, s) for p, s in ws]
    res = rng.standard_normal(8192).astype(np.float32)
    ys = [ctx.alloc(1024 * 4), ctx.upload(res), ctx.alloc(32 * 4)]
    dx, dg = ctx.upload(x), ctx.upload(gamma)
    print("case: q4 gemv multi with rms norm and in-place residual", flush=True)
    outs = [(1024, dev[0][0], dev[0][1], ys[0]), (8192, dev[1][0], dev[1][1], ys[1], ys[1]),
            (32, dev[2][0], dev[2][1], ys[2])]
    ctx.q4_gemv_multi(k, dx, outs, norm_w=dg)
    for i, ((p, s), (_, n)) in enumerate(zip(ws, shapes)):
        got = ctx.download(ys[i], (n,), np.float32).astype(np.float64)
        ref = O.q4_gemv(xn, p, s).astype(np.float64) + (res if i == 1 else 0.0)
        mag = _mag(xn, p, s) + (np.abs(res) if i == 1 else 0.0)
        print(f"out {i}: max|d|/mag {(np.abs(got - ref) / mag).max():.3e}")
        assert np.all(np.abs(got - ref) <= 1e-5 * mag + 1e-30)
    assert np.array_equal(ctx.download(dx, (k,), np.float32), x)       # x itself is not written


def test_q4_gemv_conv_fused(ctx):
    """The DeltaNet decode's input projections with the conv1d step + SiLU
    fused onto in_proj_qkv (gemv.rs:740-742,744-772,788-789,865): the
    shifted conv buffer holds the unfused projection bit for bit, and the
    activation matches the oracle's conv1d step + silu on it; the other
    outputs equal the unfused launch."""
    rng = np.random.default_rng(47)
    k = 2560
    x = rng.standard_normal(k).astype(np.float32)
    gamma = W.f16_bits(0.1 * rng.standard_normal(k).astype(np.float32))
    names = ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b")
    ws = {nm: W.q4_random_weight(*W.Q4_PROJ_SHAPES[nm], rng) for nm in names}
    dev = {nm: repack(ctx, *ws[nm]) for nm in names}
    conv_w = (0.5 * rng.standard_normal((8192, 4))).astype(np.float32)
    buf0 = rng.standard_normal((8192, 3)).astype(np.float32)
    dx, dg, dw = ctx.upload(x), ctx.upload(gamma), ctx.upload(conv_w)
    plain = {nm: ctx.alloc(W.Q4_PROJ_SHAPES[nm][1] * 4) for nm in names}
    fused = {nm: ctx.alloc(W.Q4_PROJ_SHAPES[nm][1] * 4) for nm in names}
    print("case: q4 gemv + conv1d + silu fused", flush=True)
    ctx.q4_gemv_multi(k, dx, [(W.Q4_PROJ_SHAPES[nm][1], *dev[nm], plain[nm]) for nm in names], norm_w=dg)
    dbuf = ctx.upload(buf0)
    ctx.q4_gemv_multi(k, dx, [(W.Q4_PROJ_SHAPES[nm][1], *dev[nm], fused[nm]) for nm in names], norm_w=dg,
                      conv_buf=dbuf, conv_w=dw)
    v = ctx.download(plain["in_proj_qkv"], (8192,), np.float32)
    buf = ctx.download(dbuf, (8192, 3), np.float32)
    assert np.array_equal(buf[:, :2], buf0[:, 1:]) and np.array_equal(buf[:, 2], v)
    ref_buf = buf0.copy()
    conv = O.conv1d_step(ref_buf, conv_w, v)
    ref = np.array([O.silu(float(c)) for c in conv], np.float32)
    got = ctx.download(fused["in_proj_qkv"], (8192,), np.float32)
    # silu's expf on the device and in libm differ by an ulp or so
    ulps = np.abs(got - ref) / np.spacing(np.abs(ref))
    print(f"silu: max {ulps.max():.1f} ulp")
    assert np.all(np.abs(got - ref) <= 4 * np.spacing(np.abs(ref)) + 1e-30)
    for nm in names[1:]:
        n = W.Q4_PROJ_SHAPES[nm][1]
        assert np.array_equal(ctx.download(fused[nm], (n,), np.float32), ctx.download(plain[nm], (n,), np.float32))
    with pytest.raises(M.MixerError):                   # no residual on the conv output
        ctx.q4_gemv_multi(k, dx, [(8192, *dev["in_proj_qkv"], fused["in_proj_qkv"], fused["in_proj_qkv"])],
                          conv_buf=dbuf, conv_w=dw)


@pytest.mark.parametrize("norm", [False, True])
def test_q4_gate_up(ctx, norm):
    """silu(xn Wg) * (xn Wu) (fused_gate_up_q4, gemv.rs:469-526) for the
    2560 x 9216 MLP weights, with and without the fused rms_norm."""
    rng = np.random.default_rng(41 + norm)
    k, n = 2560, 9216
    x = rng.standard_normal(k).astype(np.float32)
    gamma = W.f16_bits(0.1 * rng.standard_normal(k).astype(np.float32))
    xn = O.rms_norm(x, gamma) if norm else x
    (gp, gs), (up, us) = W.q4_random_weight(k, n, rng), W.q4_random_weight(k, n, rng)
    (gc, gg), (uc, ug) = repack(ctx, gp, gs), repack(ctx, up, us)
    out = ctx.alloc(n * 4)
    print(f"case: q4 gate/up norm={norm}", flush=True)
    ctx.q4_gate_up(k, n, ctx.upload(x), ctx.upload(gamma) if norm else None, gc, gg, uc, ug, out)
    got = ctx.download(out, (n,), np.float32).astype(np.float64)
    ref = O.q4_gate_up(xn, gp, gs, up, us).astype(np.float64)
    g = O.q4_gemv(xn, gp, gs).astype(np.float64)
    u = O.q4_gemv(xn, up, us).astype(np.float64)
    bound = 1e-5 * (1.2 * _mag(xn, gp, gs) * np.abs(u) + 1.1 * np.abs(g) * _mag(xn, up, us)) + 1e-30
    print(f"max|d| {np.abs(got - ref).max():.3e}  max|d|/bound {(np.abs(got - ref) / bound).max():.3e}")
    assert np.all(np.abs(got - ref) <= bound)


# ---- prefill: qm_rms_norm_f16 + qm_q4_gemm ----------------------------------------
def test_rms_norm_f16(ctx):
    """Per-row rms_norm (gemv.rs:571-579) into f16: within one f16 rounding of
    the oracle's fp32 rows (plus fp32 reassociation of the sum of squares)."""
    rng = np.random.default_rng(51)
    m, k = 9, 2560
    x = (2.0 * rng.standard_normal((m, k))).astype(np.float32)
    gamma = W.f16_bits(0.1 * rng.standard_normal(k).astype(np.float32))
    out = ctx.alloc(m * k * 2)
    print("case: rms_norm_f16", flush=True)
    ctx.rms_norm_f16(m, k, ctx.upload(x), ctx.upload(gamma), out)
    got = W.f16_value(ctx.download(out, (m, k), np.uint16)).astype(np.float64)
    ref = np.stack([O.rms_norm(r, gamma) for r in x]).astype(np.float64)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -10 + 1e-7)
    ctx.rms_norm_f16(m, k, ctx.upload(x), None, out)                 # plain conversion
    assert np.array_equal(ctx.download(out, (m, k), np.uint16), W.f16_bits(x))


# Tile shapes on 256 CUs: m = 1930 on the 8192-wide weight (512 tiles of
# 128 x 256) and m = 3300 on the 2560-wide one (520 tiles of 128 x 128)
# take the wide kernels, the smaller cases 64 x 128 tiles, and n = 32 the
# one-wave 16 x 32 kernel.
@pytest.mark.parametrize("name,m,mode", [("in_proj_qkv", 200, "bf16"), ("in_proj_z", 37, "bf16"),
                                         ("out_proj", 64, "residual"), ("in_proj_a", 130, "f32"),
                                         ("down_proj", 129, "residual"), ("k_proj", 1, "f32"),
                                         ("in_proj_qkv", 1930, "bf16"), ("out_proj", 3300, "residual")])
def test_q4_gemm(ctx, name, m, mode):
    """gemm_q4 (gemv.rs:529-542) on MFMA: y = x W (+ residual), x f16; bar
    |y - y_ref| <= 1e-3 * sum_k |x_k W_kj| per element (W rounded to f16 per
    element), plus the bf16 rounding of the output when it is bf16."""
    k, n = W.Q4_PROJ_SHAPES[name]
    rng = np.random.default_rng(m + n)
    packed, scales = W.q4_random_weight(k, n, rng)
    codes, gsc = repack(ctx, packed, scales)
    x16 = W.f16_bits(rng.standard_normal((m, k)).astype(np.float32))
    xv = W.f16_value(x16)
    res = rng.standard_normal((m, n)).astype(np.float32) if mode == "residual" else None
    print(f"case: q4 gemm {name} m={m} {mode}", flush=True)
    y = ctx.alloc(m * n * (2 if mode == "bf16" else 4))
    ctx.q4_gemm(m, k, n, ctx.upload(x16), codes, gsc,
                y=None if mode == "bf16" else y, y_bf16=y if mode == "bf16" else None,
                residual=None if res is None else ctx.upload(res))
    if mode == "bf16":
        got = W.bf16_value(ctx.download(y, (m, n), np.uint16)).astype(np.float64)
    else:
        got = ctx.download(y, (m, n), np.float32).astype(np.float64)
    ref = O.q4_gemm(xv, packed, scales).astype(np.float64)
    mag = np.abs(xv).astype(np.float64) @ np.abs(W.q4_dequant(packed, scales)).astype(np.float64)
    if res is not None:
        ref += res
        mag += np.abs(res)
    bound = 1e-3 * mag + (np.abs(ref) * 2.0 ** -8 if mode == "bf16" else 0.0) + 1e-30
    print(f"max|d|/bound {(np.abs(got - ref) / bound).max():.3e}  rel {np.abs(got - ref).max() / np.abs(ref).max():.3e}")
    assert np.all(np.abs(got - ref) <= bound)


# A bf16 input runs bf16 MFMA with W rounded to f16 and then to bf16: per
# term at most 2^-8 + 2^-11 of |x w| (the input itself is exact), plus the
# fp32 accumulation.
BF16_W_EPS = 2.0 ** -8 + 2.0 ** -11 + 1e-4


def _w_bf16(packed, scales):
    """W as the bf16-input GEMM multiplies it: f16(s (q - 8)), then bf16."""
    return W.bf16_value(W.bf16_bits(W.f16_value(W.f16_bits(W.q4_dequant(packed, scales)))))


@pytest.mark.parametrize("name,m", [("out_proj", 77), ("in_proj_qkv", 2000), ("down_proj", 3300),
                                    ("in_proj_a", 300)])
def test_q4_gemm_bf16_input(ctx, name, m):
    """out_proj on a mixer prefill output (bf16 [T][4096]) with the residual
    added in place (gemv.rs:1222-1223), and bf16 inputs on the other tile
    shapes (in_proj_qkv 128 x 256, down_proj 128 x 128, the 32-wide
    in_proj_a 16 x 32).  Against the oracle on the bf16
    values: |y - y_ref| <= (2^-8 + 2^-11 + 1e-4) sum_k |x_k W_kj|.  Against
    the arithmetic the kernel states (x times bf16(f16(s (q - 8))) summed in
    fp32): within 1e-5 of max |y|, where a W rounded only to f16 would differ
    by ~1e-3 of it."""
    k, n = W.Q4_PROJ_SHAPES[name]
    rng = np.random.default_rng(61 + m)
    packed, scales = W.q4_random_weight(k, n, rng)
    codes, gsc = repack(ctx, packed, scales)
    xb = W.bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    xv = W.bf16_value(xb)
    res = rng.standard_normal((m, n)).astype(np.float32)
    print(f"case: q4 gemm bf16 input, {name} m={m} residual in place", flush=True)
    y = ctx.upload(res)
    ctx.q4_gemm(m, k, n, ctx.upload(xb), codes, gsc, y=y, residual=y, x_dtype=M.QM_BF16)
    got = ctx.download(y, (m, n), np.float32).astype(np.float64)
    ref = O.q4_gemm(xv, packed, scales).astype(np.float64) + res
    bound = BF16_W_EPS * (_mag(xv, packed, scales) + np.abs(res)) + 1e-30
    print(f"max|d|/bound {(np.abs(got - ref) / bound).max():.3e}")
    assert np.all(np.abs(got - ref) <= bound)
    model = xv.astype(np.float64) @ _w_bf16(packed, scales).astype(np.float64) + res
    dev = np.abs(got - model).max() / np.abs(model - res).max()
    f16w = xv.astype(np.float64) @ W.f16_value(W.f16_bits(W.q4_dequant(packed, scales))).astype(np.float64) + res
    print(f"vs bf16-weight arithmetic {dev:.2e}, f16-weight arithmetic differs by "
          f"{np.abs(f16w - model).max() / np.abs(model - res).max():.2e}")
    assert dev <= 1e-5
    assert np.abs(f16w - model).max() / np.abs(model - res).max() > 1e-4      # the check can tell them apart


@pytest.mark.parametrize("n,m,x_dtype", [(9216, 64, "f16"), (2592, 130, "f16"), (2592, 37, "bf16"),
                                         (9216, 1000, "f16"), (9216, 1000, "bf16")])
def test_q4_gemm_gate_up(ctx, n, m, x_dtype):
    """The prefill MLP's gate/up GEMMs and silu(g) * u (gemv.rs:1231-1237)
    in one launch, written as bf16.  Bar: the GEMM bar carried through
    silu(g) * u, plus the bf16 rounding of the output.  n = 2592 ends in a
    partial 128-column tile of the 8-column device layout; m = 1000 on
    n = 9216 runs 576 workgroups, several per CU."""
    k = 2560
    rng = np.random.default_rng(n + m)
    (gp, gs), (up, us) = W.q4_random_weight(k, n, rng), W.q4_random_weight(k, n, rng)
    (gc, gg), (uc, ug) = repack(ctx, gp, gs), repack(ctx, up, us)
    xf = rng.standard_normal((m, k)).astype(np.float32)
    if x_dtype == "bf16":
        xbits, dt = W.bf16_bits(xf), M.QM_BF16
        xv = W.bf16_value(xbits)
    else:
        xbits, dt = W.f16_bits(xf), M.QM_F16
        xv = W.f16_value(xbits)
    out = ctx.alloc(m * n * 2)
    print(f"case: q4 gemm gate/up n={n} m={m} x {x_dtype}", flush=True)
    ctx.q4_gemm_gate_up(m, k, n, ctx.upload(xbits), gc, gg, uc, ug, out, x_dtype=dt)
    got = W.bf16_value(ctx.download(out, (m, n), np.uint16)).astype(np.float64)
    g = O.q4_gemm(xv, gp, gs)
    u = O.q4_gemm(xv, up, us)
    one = np.float32(1.0)
    ref = ((g / (one + np.exp(-g))) * u).astype(np.float64)
    g, u = g.astype(np.float64), u.astype(np.float64)
    eps = BF16_W_EPS if x_dtype == "bf16" else 1e-3
    bound = (eps * (1.2 * _mag(xv, gp, gs) * np.abs(u) + 1.1 * np.abs(g) * _mag(xv, up, us))
             + np.abs(ref) * 2.0 ** -8 + 1e-7)
    print(f"max|d|/bound {(np.abs(got - ref) / bound).max():.3e}")
    assert np.all(np.abs(got - ref) <= bound)


def _outlier_rows(rng, m, k, cols, scale):
    """N(0,1) rows with a few columns of |x| ~ scale (massive activations)."""
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[:, cols] *= np.float32(scale)
    return x


@pytest.mark.parametrize("scale", [3e3, 1e5])
def test_q4_gemm_gate_up_outliers(ctx, scale):
    """Outlier input channels whose gate and up products reach past f16's
    range (|silu(g) u| up to ~1e9 here): the bf16 output stays finite and
    within the bf16-input bar, and the down_proj GEMM that reads it (bf16
    input of ~1e9 in a few rows) is finite and within the same bar.  These
    sums are dominated by a few outlier terms, so the bar's per-term bound
    (W rounded to bf16) is what they are held to, without averaging."""
    k, n, m = 2560, 2592, 40
    rng = np.random.default_rng(int(scale))
    (gp, gs), (up, us) = W.q4_random_weight(k, n, rng), W.q4_random_weight(k, n, rng)
    (gc, gg), (uc, ug) = repack(ctx, gp, gs), repack(ctx, up, us)
    # bf16 input (the form whose range the kernel keeps): outliers in 3 columns of 5 rows
    xf = rng.standard_normal((m, k)).astype(np.float32)
    xf[np.ix_([0, 7, 8, 21, 39], [5, 900, 2559])] = np.float32(scale)
    xbits = W.bf16_bits(xf)
    xv = W.bf16_value(xbits)
    out = ctx.alloc(m * n * 2)
    print(f"case: q4 gemm gate/up with outliers {scale:g}", flush=True)
    ctx.q4_gemm_gate_up(m, k, n, ctx.upload(xbits), gc, gg, uc, ug, out, x_dtype=M.QM_BF16)
    hbits = ctx.download(out, (m, n), np.uint16)
    got = W.bf16_value(hbits).astype(np.float64)
    g, u = O.q4_gemm(xv, gp, gs), O.q4_gemm(xv, up, us)
    ref = ((g / (np.float32(1.0) + np.exp(-g))) * u).astype(np.float64)
    assert np.isfinite(got).all() and np.abs(ref).max() > 65504.0
    g, u = g.astype(np.float64), u.astype(np.float64)
    bound = (BF16_W_EPS * (1.2 * _mag(xv, gp, gs) * np.abs(u) + 1.1 * np.abs(g) * _mag(xv, up, us))
             + np.abs(ref) * 2.0 ** -8 + 1e-7)
    print(f"gate/up: max|h| {np.abs(ref).max():.3e}, max|d|/bound {(np.abs(got - ref) / bound).max():.3e}")
    assert np.all(np.abs(got - ref) <= bound)
    # down_proj on that bf16 intermediate (k = 2592 here), a residual as in the layer
    dp, ds = W.q4_random_weight(n, 2560, rng)
    dc, dg = repack(ctx, dp, ds)
    res = rng.standard_normal((m, 2560)).astype(np.float32)
    y = ctx.upload(res)
    ctx.q4_gemm(m, n, 2560, out, dc, dg, y=y, residual=y, x_dtype=M.QM_BF16)
    goty = ctx.download(y, (m, 2560), np.float32).astype(np.float64)
    hv = W.bf16_value(hbits)
    refy = O.q4_gemm(hv, dp, ds).astype(np.float64) + res
    boundy = BF16_W_EPS * (_mag(hv, dp, ds) + np.abs(res)) + 1e-30
    print(f"down: max|y| {np.abs(refy).max():.3e}, max|d|/bound {(np.abs(goty - refy) / boundy).max():.3e}")
    assert np.isfinite(goty).all()
    assert np.all(np.abs(goty - refy) <= boundy)


def test_q4_gemm_bf16_rows_past_f16_range_match_unscaled_rows(ctx):
    """A bf16 input row scaled by 2^20 (past f16's range, inside bf16's)
    gives exactly 2^20 times the unscaled row's result: bf16 inputs run
    bf16 MFMA with fp32 accumulation, and a power of two commutes with
    every rounding on that path."""
    k, n, m = 2560, 4096, 8
    rng = np.random.default_rng(77)
    packed, scales = W.q4_random_weight(k, n, rng)
    codes, gsc = repack(ctx, packed, scales)
    b0 = rng.standard_normal((m, k)).astype(np.float32)
    b0 = np.where(b0 < 0, -1, 1).astype(np.float32) * np.maximum(np.abs(b0), np.float32(0.01))
    base = W.bf16_value(W.bf16_bits(b0))
    big = base * np.float32(2.0 ** 20)                       # exact in bf16
    x = np.concatenate([base, big]).astype(np.float32)
    y = ctx.alloc(2 * m * n * 4)
    print("case: q4 gemm bf16 rows x 2^20", flush=True)
    ctx.q4_gemm(2 * m, k, n, ctx.upload(W.bf16_bits(x)), codes, gsc, y=y, x_dtype=M.QM_BF16)
    got = ctx.download(y, (2 * m, n), np.float32)
    assert np.isfinite(got).all()
    assert np.array_equal(got[m:], got[:m] * np.float32(2.0 ** 20))
    ref = O.q4_gemm(base, packed, scales).astype(np.float64)
    assert np.all(np.abs(got[:m] - ref) <= BF16_W_EPS * _mag(base, packed, scales) + 1e-30)


def test_q4_gemm_errors(ctx):
    w = W.q4_gemv_workload(48, 64, seed=3)
    codes, gsc = repack(ctx, w["packed"], w["scales"])
    x = ctx.alloc(4 * 48 * 2)
    y = ctx.alloc(4 * 64 * 4)
    with pytest.raises(M.MixerError) as e:             # k not a multiple of 32
        ctx.q4_gemm(4, 48, 64, x, codes, gsc, y=y)
    assert e.value.code == 4
    with pytest.raises(M.MixerError) as e:             # both outputs given
        ctx.q4_gemm(4, 32, 64, x, codes, gsc, y=y, y_bf16=y)
    assert e.value.code == 3
    with pytest.raises(M.MixerError) as e:             # x must be f16 or bf16
        ctx.q4_gemm(4, 32, 64, x, codes, gsc, y=y, x_dtype=M.QM_F32)
    assert e.value.code == 3
    with pytest.raises(M.MixerError) as e:             # gate/up: k not a multiple of 32
        ctx.q4_gemm_gate_up(4, 48, 64, x, codes, gsc, codes, gsc, y)
    assert e.value.code == 4
