"""GPU parity at the batched-decode stack workload: 32 mixer layers (24
DeltaNet + 8 GQA, pattern 3 + 1), 64 sequences at context 32768, KV cache
capacity 32896 positions (f16 [64][4][32896][256] per layer, 2.155e9
elements: offsets past 2^31 from row 128 of sequence 63's last kv head).

Two decode steps (positions 32768 and 32769) run through all 32 layers on
the device.  For sequences 0, 31 and 63 every layer is replayed on the CPU
oracle: DeltaNet layers with or_deltanet_decode_step on that sequence's
state slice (gemv.rs:744-883), GQA layers with or_attn_decode_step over the
sequence's cache read back as f32 (gemv.rs:927-1011).  Bar: max-abs <= 1e-3
on every layer output and on the final states; appended K rows within one
f16 step of the oracle's, appended V rows exact.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import load_mixer, load_oracle, load_workloads

pytestmark = pytest.mark.gpu

M = load_mixer()
O = load_oracle()
W = load_workloads()

B, CTX0, CAP, STEPS = 64, 32768, 32896, 2
N_DN, N_GQA = 24, 8
SAMPLE = (0, 31, 63)
TOL = 1e-3
S_SEQ = 32 * 128 * 128                   # state floats per sequence and layer
DN_IN = 8192 + 32 + 32 + 4096            # qkv | a | b | z per sequence
GQA_IN = 16 * 512 + 4 * 256 + 4 * 256    # q_gate | k_new | v_new per sequence
KV_SEQ = 4 * CAP * 256                   # cache elements per sequence and layer


def test_stack_b64_ctx32k_two_steps():
    rng = np.random.default_rng(44)
    dn_par = [W.dn_params(rng) for _ in range(N_DN)]
    gqa_par = [{"q_norm": W.f16_bits(0.1 * rng.standard_normal(256, dtype=np.float32)),
                "k_norm": W.f16_bits(0.1 * rng.standard_normal(256, dtype=np.float32))} for _ in range(N_GQA)]
    # per (step, layer): inputs of the 64 sequences, dn_in[s, l, b] = qkv | a | b | z of sequence b
    dn_in = rng.standard_normal((STEPS, N_DN, B, DN_IN), dtype=np.float32)
    gqa_in = rng.standard_normal((STEPS, N_GQA, B, GQA_IN), dtype=np.float32)

    def device_blocks(x, widths):
        # the entry points take each input as its own [64][width] array: per
        # (step, layer) the blocks [qkv 64 x 8192 | a 64 x 32 | ...] one after another
        out, o = [], 0
        for wd in widths:
            out.append(x[..., o:o + wd].reshape(x.shape[0], x.shape[1], -1))
            o += wd
        return np.ascontiguousarray(np.concatenate(out, axis=2))
    rope_rows = CAP
    cos, sin = M.rope_table(rope_rows)

    with M.Context(0) as c:
        bufs = []

        def alloc(nbytes):
            bufs.append(c.alloc(nbytes))
            return bufs[-1]

        try:
            print(f"case: stack B={B} ctx={CTX0} cap={CAP}: allocating and filling", flush=True)
            dpar = [{k: c.upload(p[k]) for k in ["a_log", "dt_bias", "norm_w"]} for p in dn_par]
            gpar = [{k: c.upload(p[k]) for k in ["q_norm", "k_norm"]} for p in gqa_par]
            for d in dpar + gpar:
                bufs.extend(d.values())
            rc, rs = c.upload(cos), c.upload(sin)
            bufs += [rc, rs]
            states = [alloc(B * S_SEQ * 4) for _ in range(N_DN)]
            kcs = [alloc(B * KV_SEQ * 2) for _ in range(N_GQA)]
            vcs = [alloc(B * KV_SEQ * 2) for _ in range(N_GQA)]
            for i, s in enumerate(states):
                c.fill_normal(s, M.QM_F32, B * S_SEQ, 0.0, 0.02, seed=7000 + i)
            for i, buf in enumerate(kcs + vcs):
                c.fill_normal(buf, M.QM_F16, B * KV_SEQ, 0.0, 1.0, seed=8000 + i)
            din = c.upload(device_blocks(dn_in, (8192, 32, 32, 4096)))
            gin = c.upload(device_blocks(gqa_in, (16 * 512, 4 * 256, 4 * 256)))
            bufs += [din, gin]
            dn_out = alloc(STEPS * N_DN * B * 4096 * 4)
            gqa_out = alloc(STEPS * N_GQA * B * 4096 * 4)
            c.reserve(max_batch=B, max_kv_len=CAP)
            c.sync()
            # the sampled sequences' states before the steps (2 MB each)
            s0 = {(l, b): c.download(states[l].offset(b * S_SEQ * 4), (32, 128, 128), np.float32)
                  for l in range(N_DN) for b in SAMPLE}

            for s in range(STEPS):
                pos = CTX0 + s
                print(f"case: stack step {s} (position {pos}) through 32 layers", flush=True)
                ld = lg = 0
                for layer in range(32):
                    if layer % 4 != 3:
                        base = din.offset(((s * N_DN + ld) * B * DN_IN) * 4)
                        a = base + B * 8192 * 4
                        b = a + B * 32 * 4
                        z = b + B * 32 * 4
                        p = dpar[ld]
                        c.deltanet_decode(B, M.QM_DN_POSTACT, base, None, None, a, b, p["a_log"], p["dt_bias"],
                                          z, p["norm_w"], states[ld], dn_out.offset((s * N_DN + ld) * B * 4096 * 4))
                        ld += 1
                    else:
                        base = gin.offset(((s * N_GQA + lg) * B * GQA_IN) * 4)
                        kn = base + B * 16 * 512 * 4
                        vn = kn + B * 4 * 256 * 4
                        p = gpar[lg]
                        c.gqa_decode(B, base, kn, vn, p["q_norm"], p["k_norm"], rc, rs, rope_rows, None, pos,
                                     kcs[lg], vcs[lg], CAP, gqa_out.offset((s * N_GQA + lg) * B * 4096 * 4))
                        lg += 1
                c.sync()
            got_dn = c.download(dn_out, (STEPS, N_DN, B, 4096), np.float32)
            got_gqa = c.download(gqa_out, (STEPS, N_GQA, B, 4096), np.float32)

            cfg = O.config()
            worst_dn = worst_state = 0.0
            for l in range(N_DN):
                p = dn_par[l]
                for b in SAMPLE:
                    S = s0[(l, b)].copy()
                    for s in range(STEPS):
                        x = dn_in[s, l, b]
                        ref = O.deltanet_decode_step(cfg, x[:8192], x[8192:8224], x[8224:8256], x[8256:],
                                                     np.zeros((8192, 4), np.float32), p["a_log"], p["dt_bias"],
                                                     p["norm_w"], S)
                        worst_dn = max(worst_dn, float(np.abs(got_dn[s, l, b] - ref).max()))
                    fin = c.download(states[l].offset(b * S_SEQ * 4), (32, 128, 128), np.float32)
                    worst_state = max(worst_state, float(np.abs(fin - S).max()))
            print(f"DeltaNet layers: max|dout|={worst_dn:.3e} max|dstate|={worst_state:.3e}", flush=True)
            assert worst_dn <= TOL and worst_state <= TOL

            worst_gqa = 0.0
            L = CTX0 + STEPS
            for l in range(N_GQA):
                p = gqa_par[l]
                for b in SAMPLE:
                    print(f"case: stack GQA layer {l} sequence {b} vs oracle", flush=True)
                    kdev = c.download(kcs[l].offset(b * KV_SEQ * 2), (4, CAP, 256), np.uint16)
                    vdev = c.download(vcs[l].offset(b * KV_SEQ * 2), (4, CAP, 256), np.uint16)
                    K = np.ascontiguousarray(np.transpose(W.f16_value(kdev[:, :L]), (1, 0, 2)))
                    V = np.ascontiguousarray(np.transpose(W.f16_value(vdev[:, :L]), (1, 0, 2)))
                    for s in range(STEPS):
                        x = gqa_in[s, l, b]
                        pos = CTX0 + s
                        ref = O.attn_decode_step(cfg, x[:8192], x[8192:9216], x[9216:], p["q_norm"], p["k_norm"],
                                                 cos, sin, K, V, pos, round_kv_f16=True, nthreads=8)
                        worst_gqa = max(worst_gqa, float(np.abs(got_gqa[s, l, b] - ref).max()))
                        # the appended rows (the oracle wrote its own row `pos` of K and V)
                        kg = W.f16_value(kdev[:, pos])
                        assert np.all(np.abs(kg - K[pos]) <= np.abs(K[pos]) * 2 ** -10 + 1e-7), (l, b, s)
                        assert np.array_equal(W.f16_value(vdev[:, pos]), V[pos]), (l, b, s)
                    del K, V, kdev, vdev
            print(f"GQA layers: max|dout|={worst_gqa:.3e}", flush=True)
            assert worst_gqa <= TOL
        finally:
            for buf in bufs:
                buf.close()
