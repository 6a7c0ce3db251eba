"""CPU check of the chunked (WY/UT) DeltaNet prefill algebra used by the
qm_dn_prefill_{chunk,scan,out} kernels, and of the segment form of a
sequence split (a segment maps S_in to S_in M + B; segments compose), the
algebra behind a prefill split across GPUs or segments.

The kernels evaluate, per chunk of C tokens with state S0 entering,
  A = strictly-lower(beta_i gamma_i/gamma_j k_i.k_j), T = (I + A)^-1,
  W = T diag(beta gamma) K, U~ = T diag(beta) V, P = lower(gamma_i/gamma_j q_i.k_j),
  U = U~ - W S0^T, Y = (diag(gamma) Q - P W) S0^T + P U~,
  S_C = gamma_C S0 + U^T diag(gamma_C/gamma) K,
with T built blockwise (16x16 diagonal blocks by substitution, then the
2x2-block lower-triangular inverse twice).  Here the same steps run in
float64 numpy on small dimensions and are compared with the oracle's
sequential prefill (gemv.rs:1119-1219): equal up to fp32 rounding of the
oracle.  Chunk sizes that do not divide the sequence (padded tail) and
C = 1 (the recurrence itself) are covered.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import load_oracle

O = load_oracle()


def block_tril_inverse(A: np.ndarray, blk: int) -> np.ndarray:
    """(I + A)^-1 for strictly lower A, the kernel's blocked scheme."""
    n = A.shape[0]
    T = np.zeros_like(A)
    nb = n // blk
    for b in range(nb):                           # diagonal blocks: substitution
        s = slice(b * blk, (b + 1) * blk)
        Ab = A[s, s]
        Tb = np.zeros((blk, blk))
        for i in range(blk):
            row = np.eye(blk)[i].copy()
            for j in range(i):
                row -= Ab[i, j] * Tb[j]
            Tb[i] = row
        T[s, s] = Tb
    size = blk
    while size < n:                               # merge [[X,0],[Y,Z]]^-1
        for r0 in range(0, n, 2 * size):
            X = slice(r0, r0 + size)
            Z = slice(r0 + size, r0 + 2 * size)
            T[Z, X] = -T[Z, Z] @ (A[Z, X] @ T[X, X])
        size *= 2
    return T


def chunked_prefill(q, k, v, g, beta, S0, C):
    """q,k,v [T, H, d] (q,k already normed, q scaled), g = log alpha [T, H]."""
    Tn, H, d = q.shape
    nc = -(-Tn // C)
    pad = nc * C - Tn
    q = np.concatenate([q, np.zeros((pad, H, d))])
    k = np.concatenate([k, np.zeros((pad, H, d))])
    v = np.concatenate([v, np.zeros((pad, H, d))])
    g = np.concatenate([g, np.zeros((pad, H))])
    beta = np.concatenate([beta, np.zeros((pad, H))])
    S = S0.copy()
    Y = np.zeros((nc * C, H, d))
    blk = min(16, C)
    for h in range(H):
        for c in range(nc):
            sl = slice(c * C, (c + 1) * C)
            K, Q, V = k[sl, h], q[sl, h], v[sl, h]
            G = np.cumsum(g[sl, h])
            gam = np.exp(G)
            b = beta[sl, h]
            D = np.exp(G[:, None] - G[None, :])
            A = np.tril(b[:, None] * D * (K @ K.T), -1)
            P = np.tril(D * (Q @ K.T))
            T = block_tril_inverse(A, blk) if C % blk == 0 else np.linalg.inv(np.eye(C) + A)
            W = T @ ((b * gam)[:, None] * K)
            Ut = T @ (b[:, None] * V)
            Qt = gam[:, None] * Q - P @ W
            Y0 = P @ Ut
            Kt = (np.exp(G[-1] - G))[:, None] * K
            S0h = S[h]
            U = Ut - W @ S0h.T
            Y[sl, h] = Y0 + Qt @ S0h.T
            S[h] = np.exp(G[-1]) * S0h + U.T @ Kt
    return Y[:Tn], S


def segmented_prefill(q, k, v, g, beta, S0, C, seg_chunks):
    """The two-pass segment form of a sequence split: the sequence is cut
    into segments of seg_chunks chunks; pass 1 runs every segment but the
    last from a zero state (B_s, the state rows) and from the identity with
    V = 0 (M_s, rows of the linear map), so that S_out = S_in M_s + B_s;
    the combine chains S_entry(s + 1) = S_entry(s) M_s + B_s from S0; pass
    3 reruns each segment from its entry state with the outputs."""
    Tn, H, d = q.shape
    nc = -(-Tn // C)
    NS = -(-nc // seg_chunks)

    def seg(s, S_in, vv):
        lo, hi = s * seg_chunks * C, min((s + 1) * seg_chunks * C, Tn)
        return chunked_prefill(q[lo:hi], k[lo:hi], vv[lo:hi], g[lo:hi], beta[lo:hi], S_in, C)

    Ms, Bs = [], []
    for s in range(NS - 1):
        _, B = seg(s, np.zeros_like(S0), v)
        _, Mt = seg(s, np.broadcast_to(np.eye(d), (H, d, d)).copy(), np.zeros_like(v))
        Ms.append(Mt)
        Bs.append(B)
    ent = [S0.copy()]
    for s in range(NS - 1):
        ent.append(np.einsum("hvr,hrk->hvk", ent[s], Ms[s]) + Bs[s])
    Y = np.zeros((Tn, H, d))
    for s in range(NS):
        Ys, S_last = seg(s, ent[s], v)
        lo = s * seg_chunks * C
        Y[lo:lo + Ys.shape[0]] = Ys
    return Y, S_last


def gated_norm(y, z, gw):
    inv = 1.0 / np.sqrt(np.mean(y ** 2, axis=-1, keepdims=True) + 1e-6)
    return y * inv * gw * z / (1.0 + np.exp(-z))


@pytest.mark.parametrize("Tn,C", [(150, 64), (64, 64), (37, 16), (20, 1)])
def test_chunked_algebra_matches_sequential_oracle(Tn, C):
    cfg = O.config(num_qk_heads=2, num_v_heads=4, dn_head_dim=16)
    hd, nv, nqk = 16, 4, 2
    r = np.random.default_rng(Tn + C)
    qkv = r.standard_normal((Tn, (2 * nqk + nv) * hd)).astype(np.float32)
    a = r.standard_normal((Tn, nv)).astype(np.float32)
    b = r.standard_normal((Tn, nv)).astype(np.float32)
    z = r.standard_normal((Tn, nv * hd)).astype(np.float32)
    conv_w = (0.5 * r.standard_normal(((2 * nqk + nv) * hd, 4))).astype(np.float32)
    a_log = np.log(r.uniform(0.01, 0.1, nv)).astype(np.float32)
    dt_bias = np.zeros(nv, np.float32)
    gw = (1 + 0.1 * r.standard_normal(hd)).astype(np.float16)
    S0 = (0.02 * r.standard_normal((nv, hd, hd))).astype(np.float32)
    buf0 = (0.3 * r.standard_normal(((2 * nqk + nv) * hd, 3))).astype(np.float32)

    S_or, buf = S0.copy(), buf0.copy()
    ref = O.deltanet_prefill(cfg, qkv, a, b, z, conv_w, a_log, dt_bias, gw.view(np.uint16), S_or, buf)

    # activation exactly as the chunk kernel: causal conv with the buffer, SiLU, L2 norm, q scale
    x = np.vstack([buf0.T.astype(np.float64), qkv.astype(np.float64)])
    conv = sum(x[j:j + Tn] * conv_w[:, j].astype(np.float64) for j in range(4))
    act = conv / (1 + np.exp(-conv))
    q = act[:, :nqk * hd].reshape(Tn, nqk, hd)
    k = act[:, nqk * hd:2 * nqk * hd].reshape(Tn, nqk, hd)
    v = act[:, 2 * nqk * hd:].reshape(Tn, nv, hd)
    q = q / np.linalg.norm(q, axis=-1, keepdims=True) / np.sqrt(hd)
    k = k / np.linalg.norm(k, axis=-1, keepdims=True)
    rep = nv // nqk
    q, k = np.repeat(q, rep, axis=1), np.repeat(k, rep, axis=1)     # v head h -> qk head h // 2
    g = -np.exp(a_log.astype(np.float64)) * np.log1p(np.exp(a.astype(np.float64) + dt_bias))
    beta = 1 / (1 + np.exp(-b.astype(np.float64)))
    Y, S = chunked_prefill(q, k, v, g, beta, S0.astype(np.float64), C)
    out = gated_norm(Y, z.reshape(Tn, nv, hd).astype(np.float64), gw.astype(np.float64)).reshape(Tn, -1)
    assert np.abs(out - ref).max() < 2e-4
    assert np.abs(S - S_or).max() < 2e-5
    assert np.array_equal(buf, qkv[-3:].T)
    # the segment form (pass 1 maps, combine, pass 3) gives the same outputs and state
    for seg_chunks in (1, 2, 3):
        Ys, Ss = segmented_prefill(q, k, v, g, beta, S0.astype(np.float64), C, seg_chunks)
        assert np.abs(Ys - Y).max() < 1e-9 and np.abs(Ss - S).max() < 1e-9


def test_segment_maps_compose():
    """S_out = S_in M + B over a segment holds for any entering state, and
    two segments compose as (M1 M2, B1 M2 + B2)."""
    r = np.random.default_rng(5)
    Tn, H, d, C = 96, 2, 8, 16
    q = r.standard_normal((Tn, H, d)); q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k = r.standard_normal((Tn, H, d)); k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = r.standard_normal((Tn, H, d))
    g = -r.uniform(0.0, 0.2, (Tn, H))
    beta = r.uniform(0.0, 1.0, (Tn, H))
    eye = np.broadcast_to(np.eye(d), (H, d, d)).copy()
    zero = np.zeros((H, d, d))
    half = Tn // 2
    _, M1 = chunked_prefill(q[:half], k[:half], 0 * v[:half], g[:half], beta[:half], eye, C)
    _, B1 = chunked_prefill(q[:half], k[:half], v[:half], g[:half], beta[:half], zero, C)
    _, M2 = chunked_prefill(q[half:], k[half:], 0 * v[half:], g[half:], beta[half:], eye, C)
    _, B2 = chunked_prefill(q[half:], k[half:], v[half:], g[half:], beta[half:], zero, C)
    S_in = r.standard_normal((H, d, d))
    _, S_direct = chunked_prefill(q, k, v, g, beta, S_in, C)
    S_two = np.einsum("hvr,hrk->hvk", np.einsum("hvr,hrk->hvk", S_in, M1) + B1, M2) + B2
    S_composed = np.einsum("hvr,hrk->hvk", S_in, np.einsum("hvr,hrk->hvk", M1, M2)) + \
        np.einsum("hvr,hrk->hvk", B1, M2) + B2
    assert np.abs(S_two - S_direct).max() < 1e-10
    assert np.abs(S_composed - S_direct).max() < 1e-10
    # M does not depend on V, and is not the identity (the map really acts)
    _, M1b = chunked_prefill(q[:half], k[:half], 0 * v[:half] + 0, g[:half], beta[:half], eye, C)
    assert np.array_equal(M1, M1b) and np.abs(M1 - eye).max() > 1e-2


def test_blocked_inverse_is_the_inverse():
    r = np.random.default_rng(0)
    A = np.tril(r.standard_normal((64, 64)) * 0.3, -1)
    T = block_tril_inverse(A, 16)
    assert np.abs(T @ (np.eye(64) + A) - np.eye(64)).max() < 1e-10
