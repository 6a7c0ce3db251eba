"""GPU parity: the vocabulary side of a step, qm_q4_embed and qm_q4_lm_head,
vs the CPU oracle (embed_lookup_q4, gemv.rs:544-563; the final rms_norm and
lm_head_parallel's Q4 arm, gemv.rs:571-579,678-708).

Embedding rows are exact (s * (q - 8) in f32).  lm_head sums in another
fixed order than the reference's row loop: per logit
|l - l_ref| <= 1e-5 * sum_j |xn_j W_vj| (fp32 reassociation over the
hidden columns), and bit-identical results run to run.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import load_mixer, load_oracle, load_workloads

pytestmark = pytest.mark.gpu

M = load_mixer()
O = load_oracle()
W = load_workloads()


def _embed(vocab, hidden, seed):
    rng = np.random.default_rng(seed)
    packed, scales = W.q4_random_weight(vocab, hidden, rng, scale=0.02)
    return rng, packed, scales


def _lm_head(ctx, x, gamma, packed, scales):
    vocab, hidden = packed.shape[0], packed.shape[1] * 2
    out = ctx.alloc(vocab * 4)
    ctx.q4_lm_head(vocab, hidden, ctx.upload(x), None if gamma is None else ctx.upload(gamma),
                   ctx.upload(packed), ctx.upload(scales), out)
    return ctx.download(out, (vocab,), np.float32)


def test_lm_head_full_vocab_with_final_norm(ctx):
    """248,320 x 2560 with the final rms_norm (1 + gamma) fused."""
    vocab, hidden = 248320, 2560
    rng, packed, scales = _embed(vocab, hidden, 81)
    x = (3.0 * rng.standard_normal(hidden)).astype(np.float32)
    gamma = W.f16_bits(0.1 * rng.standard_normal(hidden).astype(np.float32))
    print("case: lm_head 248320 x 2560, final norm", flush=True)
    got = _lm_head(ctx, x, gamma, packed, scales).astype(np.float64)
    xn = O.rms_norm(x, gamma)
    ref = O.q4_lm_head(xn, packed, scales).astype(np.float64)
    mag = np.abs(W.q4_dequant(packed, scales)).astype(np.float64) @ np.abs(xn).astype(np.float64)
    print(f"max|d|/mag {(np.abs(got - ref) / mag).max():.3e}")
    assert np.all(np.abs(got - ref) <= 1e-5 * mag)
    assert np.array_equal(got, _lm_head(ctx, x, gamma, packed, scales).astype(np.float64))


@pytest.mark.parametrize("vocab,hidden", [(1001, 2560), (4097, 512), (333, 1024), (2050, 4096), (7, 8192), (31, 2560)])
def test_lm_head_shapes(ctx, vocab, hidden):
    """Ragged vocab (not a multiple of the 32-row super-batches, fewer rows
    than one), workgroups of 64 to 1024 threads, and no norm."""
    rng, packed, scales = _embed(vocab, hidden, vocab + hidden)
    x = rng.standard_normal(hidden).astype(np.float32)
    print(f"case: lm_head {vocab} x {hidden}", flush=True)
    got = _lm_head(ctx, x, None, packed, scales).astype(np.float64)
    ref = O.q4_lm_head(x, packed, scales).astype(np.float64)
    mag = np.abs(W.q4_dequant(packed, scales)).astype(np.float64) @ np.abs(x).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 1e-5 * mag)


def test_embed_rows_exact(ctx):
    vocab, hidden = 248320, 2560
    _, packed, scales = _embed(vocab, hidden, 82)
    ids = np.array([0, vocab - 1, 5, 5, 123456, 77, 200000], np.int32)
    out = ctx.alloc(len(ids) * hidden * 4)
    print("case: embed 7 ids", flush=True)
    ctx.q4_embed(len(ids), vocab, hidden, ctx.upload(ids), ctx.upload(packed), ctx.upload(scales), out)
    got = ctx.download(out, (len(ids), hidden), np.float32)
    for r, v in enumerate(ids):
        assert np.array_equal(got[r], O.q4_embed(packed, scales, int(v)))


def test_embed_out_of_range_and_errors(ctx):
    vocab, hidden = 64, 96
    _, packed, scales = _embed(vocab, hidden, 83)
    ids = np.array([3, vocab, -1], np.int32)
    dp, ds = ctx.upload(packed), ctx.upload(scales)
    out = ctx.alloc(3 * hidden * 4)
    ctx.q4_embed(3, vocab, hidden, ctx.upload(ids), dp, ds, out)
    got = ctx.download(out, (3, hidden), np.float32)
    assert np.array_equal(got[0], O.q4_embed(packed, scales, 3))
    assert np.all(np.isnan(got[1])) and np.all(np.isnan(got[2]))
    with pytest.raises(M.MixerError) as e:
        ctx.q4_embed(3, vocab, 100, ctx.upload(ids), dp, ds, out)
    assert e.value.code == 4
    for hidden in (2080, 8704):           # not a multiple of 512; more than 8192
        with pytest.raises(M.MixerError) as e:
            ctx.q4_lm_head(vocab, hidden, out, None, dp, ds, out)
        assert e.value.code == 4
