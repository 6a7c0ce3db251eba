"""GPU: the allocation-free GQA decode entry (qm_gqa_decode_noalloc) against
qm_gqa_decode on the same inputs, through the C ABI.

Both run the same kernels with the same launch shapes, so the outputs and
the appended cache rows must be bit-identical; the first call is also held
to the oracle's bar (max-abs <= 1e-3, gemv.rs:927-1011).  Two calls in a row,
the second with a smaller input (fewer sequences, a shorter context), check
that the shared scratch carries nothing over.  A call whose partials exceed
the fixed scratch is refused before anything is enqueued.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import load_mixer, load_oracle, load_workloads

pytestmark = pytest.mark.gpu

M = load_mixer()
O = load_oracle()
W = load_workloads()


def _both(c, w, batch, pos, rope_rows, chunk):
    cos, sin = M.rope_table(rope_rows)
    keys = ["q_gate", "k_new", "v_new", "q_norm", "k_norm", "k_cache", "v_cache"]
    d = {k: c.upload(w[k]) for k in keys}
    rc, rs = c.upload(cos), c.upload(sin)
    outs = {}
    c.set_option(M.QM_OPT_GQA_DECODE_CHUNK, chunk)
    try:
        for name in ("regular", "noalloc"):
            out = c.alloc(batch * 16 * 256 * 4)
            c.fill_normal(out, M.QM_F32, batch * 16 * 256, 0.0, 1.0, seed=3)
            fn = c.gqa_decode if name == "regular" else c.gqa_decode_noalloc
            fn(batch, d["q_gate"], d["k_new"], d["v_new"], d["q_norm"], d["k_norm"], rc, rs, rope_rows, None, pos,
               d["k_cache"], d["v_cache"], w["cap"], out)
            c.sync()
            outs[name] = (c.download(out, (batch, 16, 256), np.float32),
                          c.download(d["k_cache"], w["k_cache"].shape, np.uint16),
                          c.download(d["v_cache"], w["v_cache"].shape, np.uint16))
    finally:
        c.set_option(M.QM_OPT_GQA_DECODE_CHUNK, 0)
    return outs


def test_noalloc_matches_regular_entry_twice_second_smaller():
    with M.Context(0) as c:
        # first call: 4 sequences at position 3000 (automatic split size)
        print("case: gqa decode noalloc B=4 pos=3000", flush=True)
        w = W.gqa_decode_workload(3000, 4, seed=21)
        o = _both(c, w, 4, 3000, 3001, 0)
        for a, b in zip(o["regular"], o["noalloc"]):
            assert np.array_equal(a, b)
        cfg = O.config()
        cos, sin = O.rope_table(3001)
        for bi in (0, 3):
            K = np.ascontiguousarray(np.transpose(W.f16_value(w["k_cache"][bi, :, :3001]), (1, 0, 2)))
            V = np.ascontiguousarray(np.transpose(W.f16_value(w["v_cache"][bi, :, :3001]), (1, 0, 2)))
            ref = O.attn_decode_step(cfg, w["q_gate"][bi].ravel(), w["k_new"][bi].ravel(), w["v_new"][bi].ravel(),
                                     w["q_norm"], w["k_norm"], cos, sin, K, V, 3000, round_kv_f16=True, nthreads=8)
            assert np.abs(o["noalloc"][0][bi].ravel() - ref).max() <= 1e-3
        # second call, smaller: 2 sequences at position 700, 64-key splits (11 partials per head group)
        print("case: gqa decode noalloc B=2 pos=700 chunk=64", flush=True)
        w2 = W.gqa_decode_workload(700, 2, seed=22)
        o2 = _both(c, w2, 2, 700, 701, 64)
        for a, b in zip(o2["regular"], o2["noalloc"]):
            assert np.array_equal(a, b)


def test_noalloc_refuses_partials_beyond_the_scratch():
    with M.Context(0) as c:
        # 8 sequences, 20000 keys in 64-key splits: 8 x 4 x 313 partials = 41.7 MB > 32 MiB
        print("case: gqa decode noalloc over the scratch size (refused on the host)", flush=True)
        w = W.gqa_decode_workload(19999, 8, cap=20000, seed=23)
        cos, sin = M.rope_table(20000)
        keys = ["q_gate", "k_new", "v_new", "q_norm", "k_norm", "k_cache", "v_cache"]
        d = {k: c.upload(w[k]) for k in keys}
        rc, rs = c.upload(cos), c.upload(sin)
        out = c.alloc(8 * 16 * 256 * 4)
        c.set_option(M.QM_OPT_GQA_DECODE_CHUNK, 64)
        try:
            with pytest.raises(M.MixerError) as e:
                c.gqa_decode_noalloc(8, d["q_gate"], d["k_new"], d["v_new"], d["q_norm"], d["k_norm"], rc, rs,
                                     20000, None, 19999, d["k_cache"], d["v_cache"], w["cap"], out)
            assert e.value.code == 9          # QM_ERR_WORKSPACE
        finally:
            c.set_option(M.QM_OPT_GQA_DECODE_CHUNK, 0)


def test_noalloc_scratch_is_held_by_one_context_per_gpu():
    """A second context on the same GPU is refused while the first holds the
    scratch (their calls could overlap and race), and may use it once the
    first is destroyed."""
    w = W.gqa_decode_workload(300, 1, seed=24)
    cos, sin = M.rope_table(301)

    def call(c):
        keys = ["q_gate", "k_new", "v_new", "q_norm", "k_norm", "k_cache", "v_cache"]
        d = {k: c.upload(w[k]) for k in keys}
        rc, rs = c.upload(cos), c.upload(sin)
        out = c.alloc(16 * 256 * 4)
        c.gqa_decode_noalloc(1, d["q_gate"], d["k_new"], d["v_new"], d["q_norm"], d["k_norm"], rc, rs, 301, None,
                             300, d["k_cache"], d["v_cache"], w["cap"], out)
        c.sync()
        return c.download(out, (16, 256), np.float32)

    print("case: gqa decode noalloc, two contexts on one GPU", flush=True)
    a = M.Context(0)
    b = M.Context(0)
    try:
        ra = call(a)
        with pytest.raises(M.MixerError) as e:
            call(b)
        assert e.value.code == 9          # QM_ERR_WORKSPACE
        ra2 = call(a)                     # the holder keeps working
        assert np.array_equal(ra, ra2)
    finally:
        a.close()
    try:
        assert np.array_equal(call(b), ra)
    finally:
        b.close()


def test_noalloc_captured_without_reserve_replays_like_eager():
    """Captured into a HIP graph on a fresh context that never called
    qm_reserve (the callers this entry is for), the replays equal the eager
    call bit for bit, with eager work and synchronisation between them."""
    with M.Context(0) as c:
        print("case: gqa decode noalloc captured on an unreserved context, B=2 pos=2000", flush=True)
        w = W.gqa_decode_workload(2000, 2, seed=25)
        cos, sin = M.rope_table(2001)
        keys = ["q_gate", "k_new", "v_new", "q_norm", "k_norm", "k_cache", "v_cache"]
        d = {k: c.upload(w[k]) for k in keys}
        rc, rs = c.upload(cos), c.upload(sin)
        out = c.alloc(2 * 16 * 256 * 4)

        def call():
            c.gqa_decode_noalloc(2, d["q_gate"], d["k_new"], d["v_new"], d["q_norm"], d["k_norm"], rc, rs, 2001,
                                 None, 2000, d["k_cache"], d["v_cache"], w["cap"], out)

        c.graph_begin()
        call()
        g = c.graph_end()
        call()
        c.sync()
        ref = c.download(out, (2, 16, 256), np.float32)
        for rep in range(4):
            c.fill_normal(out, M.QM_F32, 2 * 16 * 256, 0.0, 1.0, seed=rep)
            c.upload(w["q_gate"], d["q_gate"])      # eager work between the replays
            c.sync()
            g.launch()
            c.sync()
            assert np.array_equal(c.download(out, (2, 16, 256), np.float32), ref), rep
        g.close()
