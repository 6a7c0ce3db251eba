// dn_prefill.hip -- Gated DeltaNet chunked prefill (chunk 64) for gfx950.
//
// Replaces the sequential mixer loop of prefill_deltanet_layer
// (gemv.rs:1119-1219): the same recurrence as seq_len decode steps, in the
// chunked WY/UT form.  For a chunk with state S0 entering (S is
// [v-row][k-col], gemv.rs:813), cumulative decays gamma_i = prod_{j<=i}
// alpha_j (G = log gamma) and
//   A_ij = beta_i (gamma_i/gamma_j) k_i.k_j  (j < i),  T = (I + A)^-1,
//   W = T diag(beta gamma) K,  U~ = T diag(beta) V,
//   P_ij = (gamma_i/gamma_j) q_i.k_j  (j <= i),
// the token updates collapse to
//   U = U~ - W S0^T                      (the delta-rule residuals)
//   Y = (diag(gamma) Q - P W) S0^T + P U~  (outputs y_i = S_i q_i)
//   S_C = gamma_C S0 + U^T diag(gamma_C/gamma) K.
//
// Three kernels:
//   qm_dn_prefill_chunk  everything that does not depend on S0, fully
//                        parallel over (chunk, qk-head; its two v-heads in
//                        turn, two workgroups per CU): the conv1d + SiLU +
//                        L2 norm of the chunk's q, k, v and the gates into
//                        LDS, KK^T / QK^T on MFMA, [W | U~] by block forward
//                        substitution (16x16 diagonal inverses by
//                        substitution in fp32, the off-diagonal corrections
//                        on MFMA), Q~ = diag(gamma)Q - PW and Y0 = PU~, all
//                        products on f16 MFMA;
//   qm_dn_prefill_scan   the sequential part: one 4-wave workgroup per
//                        (v-head, 16 state rows) with its rows of the fp32
//                        state in registers, two f16 MFMA GEMMs per chunk
//                        split over the waves, and the slice's outputs
//                        Y = Y0 + Q~ S_c^T from each chunk's entry state
//                        S_c (or the exact fp32 path, see the guard);
//   qm_dn_prefill_out    the gated RMSNorm over the head's 128 rows of Y,
//                        fully parallel over (chunk, v-head), and the conv
//                        buffer update.
#include "qm_device.h"
#include "qm_kernel_args.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

#define CHK QM_DN_CHUNK

QM_DEV half8 cat8(half4 a, half4 b) {
    return half8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// max(m, |v0|, .., |v3|): the running largest magnitude that an f16
// conversion must hold.  IEEE maximum (NaN-propagating, so a NaN also fails
// the f16 range check) compiles to two v_maximum3_f32 with abs modifiers;
// fmaxf's maxNum needs a canonicalising max per MFMA result first.
QM_DEV float max_abs(float m, float a) { return __builtin_elementwise_maximum(m, fabsf(a)); }
QM_DEV float max_abs4(float m, floatx4 v) {
    return max_abs(max_abs(max_abs(max_abs(m, v[0]), v[1]), v[2]), v[3]);
}

QM_DEV half4 to_half4(floatx4 v) {
    half4 r;
    r[0] = (_Float16)v[0]; r[1] = (_Float16)v[1]; r[2] = (_Float16)v[2]; r[3] = (_Float16)v[3];
    return r;
}

// LDS of the chunk kernel for the v-head it is working on (the two v-heads
// of a qk-head take it in turn).
struct ChunkHeadLds {
    _Float16 Vs[CHK][136];                         // v row-major
    _Float16 pm[CHK][72];                          // P (lower, incl. diagonal)
    _Float16 am[CHK][72];                          // -A (strictly lower), the sign the solve uses
    _Float16 Td[4][16][24];                        // (I + A_bb)^-1
};

// Per-v-head gates of the chunk (both heads' are formed in the first phase).
struct ChunkGates {
    __attribute__((aligned(16))) float Gs[CHK];    // in-chunk cumulative log decay G_i
    float Bs[CHK], Eg[CHK], BG[CHK];               // beta_i, gamma_i, beta_i gamma_i
    __attribute__((aligned(16))) float Kd[CHK];    // gamma_C / gamma_i
};

// Phase 0 of the chunk kernel for NP parts of 128 channels: causal conv1d
// (gemv.rs:1132-1147), SiLU (:1149) and, for the first NQK parts (q, then k),
// the per-head L2 norm and q scale (:1151-1156), f16 into dst[part].  Thread
// (cg, tg) = (tid & 15, tid >> 4) owns channels chb[part] .. +7 for tokens
// 4tg .. 4tg+3: the 16 lanes of a DPP row share the tokens, so the L2 norm is
// a row reduction.  All 7 NP raw rows the thread needs are loaded at
// clamped, always valid rows before any arithmetic; rows before the sequence
// come from the conv buffer, and the tokens past it are zeroed at the end.
// The gate inputs of both v-heads (waves 0 and 1) are requested after the
// rows when `gates` is set (a wave's loads return in issue order, and these
// 4-byte loads touch one cache line per token).  vm gets each v channel's
// max |v| over the valid tokens.
template <int NP, int NQK>
QM_DEV void chunk_prep(const DnPrefillArgs& A, const int (&chb)[NP], _Float16 (*const (&dst)[NP])[136],
                       int qkh, int t0, int c, bool tail, bool gates, float& ga, float& gb, float (&vm)[8]) {
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));                 // no row addresses shared with another call's
    const int cg = tid & 15, tg = tid >> 4;
    uint4 u[NP][7];
#pragma unroll
    for (int part = 0; part < NP; ++part)
#pragma unroll
        for (int r = 0; r < 7; ++r) {
            const int t = min(max(t0 + 4 * tg - 3 + r, 0), A.T - 1);
            u[part][r] = *reinterpret_cast<const uint4*>(A.qkv + (size_t)t * QM_DN_QKV_DIM + chb[part]);
        }
    float4 wt[8], wn[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) wt[e] = ld4(A.conv_w + (size_t)(chb[0] + e) * 4);
    if (gates && tid < 2 * CHK) {
        const int t = min(t0 + (tid & (CHK - 1)), A.T - 1);
        const int h = 2 * qkh + (tid >> 6);
        ga = A.a[(size_t)t * QM_DN_V_HEADS + h];
        gb = A.b[(size_t)t * QM_DN_V_HEADS + h];
    }
#pragma unroll
    for (int part = 0; part < NP; ++part) {
        const int ch0 = chb[part];
        if (part + 1 < NP) {                       // next part's taps while this one computes
#pragma unroll
            for (int e = 0; e < 8; ++e) wn[e] = ld4(A.conv_w + (size_t)(chb[part + 1] + e) * 4);
        }
        float x[7][8];
#pragma unroll
        for (int r = 0; r < 7; ++r) {
            const uint32_t wv[4] = {u[part][r].x, u[part][r].y, u[part][r].z, u[part][r].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[r][2 * e] = bf16_to_f32((uint16_t)(wv[e] & 0xffffu));
                x[r][2 * e + 1] = bf16_to_f32((uint16_t)(wv[e] >> 16));
            }
        }
        // the masks are wave-uniform branches: interior chunks skip them
        if (c == 0) {                              // x_{-3..-1} from the conv buffer
            asm volatile("" ::: "memory");        // keep these loads inside the branch
#pragma unroll
            for (int r = 0; r < 3; ++r) {
                const int t = 4 * tg - 3 + r;
                const int tb = min(t, -1);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float cbv = A.conv_buf[(size_t)(ch0 + e) * 3 + 3 + tb];
                    x[r][e] = t < 0 ? cbv : x[r][e];
                }
            }
            // the selects complete here, inside the branch: no load of it
            // is then pending where the paths join, and other chunks'
            // arithmetic waits only for the rows it uses
#pragma unroll
            for (int r = 0; r < 3; ++r)
#pragma unroll
                for (int e = 0; e < 8; ++e) asm volatile("" : "+v"(x[r][e]));
        }
        const float scale = part == 0 ? 1.0f / sqrtf((float)QM_DN_HD) : 1.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int tok = 4 * tg + j;
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                // gemv.rs:1134-1139: taps oldest first, then the new token
                float sacc = x[j][e] * wt[e].x;
                sacc = fmaf(x[j + 1][e], wt[e].y, sacc);
                sacc = fmaf(x[j + 2][e], wt[e].z, sacc);
                sacc = fmaf(x[j + 3][e], wt[e].w, sacc);
                v[e] = silu_fast(sacc);
            }
            // (tail is wave-uniform: interior chunks take every token)
            if (part >= NQK && (!tail || t0 + tok < A.T)) {
#pragma unroll
                for (int e = 0; e < 8; ++e) vm[e] = max_abs(vm[e], v[e]);
            }
            if (part < NQK) {
                // x /= ||x|| when ||x|| > 1e-12, q *= 1/sqrt(128)
                float ss = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) ss = fmaf(v[e], v[e], ss);
                ss = row_sum16(ss);
                const float f = (ss > 1e-24f ? __builtin_amdgcn_rsqf(ss) : 1.0f) * scale;
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] *= f;
            }
            half8 hv;
#pragma unroll
            for (int e = 0; e < 8; ++e) hv[e] = (_Float16)v[e];
            *reinterpret_cast<half8*>(&dst[part][tok][8 * cg]) = hv;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) wt[e] = wn[e];
    }
    if (tail) {
        // Tokens past the sequence read clamped rows above; their rows are
        // zeroed here (a token's conv and norm involve only itself and
        // earlier rows, so no valid token saw them).
#pragma unroll
        for (int part = 0; part < NP; ++part)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (t0 + 4 * tg + j >= A.T) *reinterpret_cast<half8*>(&dst[part][4 * tg + j][8 * cg]) = half8{};
    }
}

// The v-channel maxima of one v part, reduced over the wave's 64 tokens:
// lanes cg, cg+16, cg+32, cg+48 hold the same channels.  Wave w's result
// goes to red[w][channel]; om gets the largest.
QM_DEV void chunk_vmax(float (&vm)[8], float (*red)[QM_DN_HD], float& om) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, cg = threadIdx.x & 15;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(vm[e]), __float_as_uint(vm[e]), false, false);
        const float m16 = __builtin_elementwise_maximum(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
        const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(m16), __float_as_uint(m16), false, false);
        vm[e] = __builtin_elementwise_maximum(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
        om = __builtin_elementwise_maximum(om, vm[e]);
    }
    if ((lane >> 4) == 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) red[w][8 * cg + e] = vm[e];
    }
}

// ============================================================================
// 2. chunk: per (chunk, qk-head), everything independent of the entering state
// ============================================================================
// One 4-wave workgroup takes the qk-head's two v-heads 2 qkh and 2 qkh + 1
// in turn: q and k (shared by both), v of the first head and both heads'
// gates are formed first, the second head's v once the first head is done
// with the per-head LDS.  At ~79 KB of LDS two workgroups share a CU, so
// one's stalls (loads, barriers, MFMA and LDS latency) can be filled by the
// other's work; an 8-wave workgroup doing both heads at once (119 KB, one per
// CU) measured 74.5 us against 71 us for a 4096-token layer.
// [W | U~] = (I + A)^-1 [diag(beta gamma) K | diag(beta) V] is solved by block
// forward substitution over the four 16-token blocks b:
//   R_b = B_b - sum_{k<b} A_bk X_k,  X_b = T_bb R_b,  T_bb = (I + A_bb)^-1,
// with the 16x16 diagonal inverses by substitution in fp32 and the products on
// v_mfma_f32_16x16x16_f16.  Each wave owns 4 of the 16 column tiles (k-col
// tiles 2w, 2w+1 of W and v-col tiles 2w, 2w+1 of U~) for every block, and
// an X_k fragment (4 consecutive tokens of one column per lane) is already
// the B operand of the next block's correction, so the solve needs no
// workgroup barrier.
extern "C" __global__ __launch_bounds__(QM_DN_CHUNK_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
void qm_dn_prefill_chunk(DnPrefillArgs A) {
    __shared__ _Float16 Qs[CHK][136];              // q row-major
    __shared__ _Float16 Ks[CHK][136];              // k row-major
    __shared__ ChunkHeadLds H;                     // the v-head being worked on
    __shared__ ChunkGates gts[2];
    __shared__ float vred[2][4][QM_DN_HD];         // per head and wave: max |v| per channel
    __shared__ int vbad[2];                        // per head: an f16 operand would overflow

    const int tid = threadIdx.x;
    // GVA: v-heads 2 qkh and 2 qkh + 1 read qk-head qkh (gemv.rs:1160)
    const int c = blockIdx.x / QM_DN_QK_HEADS, qkh = blockIdx.x % QM_DN_QK_HEADS;
    const int t0 = c * CHK;
    const bool tail = t0 + CHK > A.T;              // last chunk, partly past the sequence
    _Float16 (&Vs)[CHK][136] = H.Vs;
    _Float16 (&Pm)[CHK][72] = H.pm;
    _Float16 (&Am)[CHK][72] = H.am;
    _Float16 (&Td)[4][16][24] = H.Td;
    if (tid < 2) vbad[tid] = 0;
    // the gate parameters of the v-head whose gates this wave forms (waves 0, 1)
    const int hg = 2 * qkh + ((tid >> 6) & 1);
    const float a_log_g = A.a_log[hg], dt_bias_g = A.dt_bias[hg];
    float om_v0 = 0.0f;                            // the first head's largest |v|

    // ---- 0. q, k and the first head's v, and both heads' gates (gemv.rs:1171-1172)
    {
        const int cg = tid & 15;
        const int chb[2] = {qkh * QM_DN_HD + 8 * cg, QM_DN_QK_DIM + qkh * QM_DN_HD + 8 * cg};
        _Float16 (*const dst[2])[136] = {Qs, Ks};
        const int chv[1] = {2 * QM_DN_QK_DIM + (2 * qkh) * QM_DN_HD + 8 * cg};
        _Float16 (*const dsv[1])[136] = {Vs};
        float ga = 0.0f, gb = 0.0f, vm[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) vm[e] = 0.0f;
        chunk_prep<2, 2>(A, chb, dst, qkh, t0, c, tail, true, ga, gb, vm);
        chunk_prep<1, 0>(A, chv, dsv, qkh, t0, c, tail, false, ga, gb, vm);
        chunk_vmax(vm, vred[0], om_v0);
        if (tid < 2 * CHK) {
            // log alpha = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b);
            // padded tokens get alpha = 1, beta = 0 (no effect on the state);
            // then the inclusive prefix sum over the chunk (one wave per head)
            // (the hardware transcendentals, a few ulp from libm)
            const int hh = tid >> 6, i = tid & (CHK - 1);
            ChunkGates& G = gts[hh];
            float g = 0.0f, be = 0.0f;
            // opaque here, so that the compiler does not start this
            // arithmetic next to the loads (a wait for every earlier load)
            asm volatile("" : "+v"(ga), "+v"(gb));
            if (t0 + i < A.T) {
                g = -exp_fast(a_log_g) * softplus_fast(ga + dt_bias_g);
                be = sigmoid_fast(gb);
            }
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const float o = __shfl_up(g, off);
                if (i >= off) g += o;
            }
            const float eg = exp_fast(g);
            G.Gs[i] = g;
            G.Bs[i] = be;
            G.Eg[i] = eg;                          // gamma_i
            G.BG[i] = be * eg;                     // beta_i gamma_i
        }
    }
    __syncthreads();
    if (tid < 2 * CHK) {
        ChunkGates& G = gts[tid >> 6];
        const int i = tid & (CHK - 1);
        G.Kd[i] = exp_fast(G.Gs[CHK - 1] - G.Gs[i]);   // gamma_C / gamma_i
    }

#pragma unroll 1
    for (int hh = 0; hh < 2; ++hh) {
        // The thread's indices, re-derived from an opaque copy in each pass:
        // otherwise the compiler computes every lane-dependent address and
        // constant of the body once, ahead of the loop, and keeps them all
        // live across both passes (it spilled them).
        int tid = threadIdx.x;
        asm volatile("" : "+v"(tid));
        const int lane = tid & 63, lr = lane & 15, lq = lane >> 4;
        const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave
        const int h = 2 * qkh + hh;
        const size_t hc = (size_t)h * A.nc + c;
        const ChunkGates& G = gts[hh];
        // largest magnitude this thread converts to an f16 operand in the
        // solve (q, k, A, P and K~ are bounded by the normalisation)
        float om = hh == 0 ? om_v0 : 0.0f;
        if (hh == 1) {
            // the second head's v, into the per-head LDS the first head has
            // finished with (the barrier after its statistics)
            const int cg = tid & 15;
            const int chb[1] = {2 * QM_DN_QK_DIM + h * QM_DN_HD + 8 * cg};
            _Float16 (*const dst[1])[136] = {Vs};
            float ga = 0.0f, gb = 0.0f, vm[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) vm[e] = 0.0f;
            chunk_prep<1, 0>(A, chb, dst, qkh, t0, c, tail, false, ga, gb, vm);
            chunk_vmax(vm, vred[1], om);
            __syncthreads();
        }

        // ---- 1. KK^T and QK^T (16x16x32 f16), masked and decayed -> -A, P (f16).
        //      Computed transposed, C = K_j K_i^T and K_j Q_i^T: lane (lr, lq)
        //      then holds row i = 16 rt + lr, columns 16j + 4lq .. +3, one
        //      8-byte store per matrix and tile.  Decays exp(G_i - G_jj) on
        //      v_exp_f32 with the exponent clamped at 0 (the masked upper
        //      part).  Row tile rt has rt + 1 column tiles; the second head
        //      takes its row tiles in the opposite order, so that every wave
        //      has five tiles over the two heads.
        {
            const int rt = hh ? 3 - w : w;
            const int i = 16 * rt + lr;
            const float gi = G.Gs[i], bi = G.Bs[i];
            half8 bk[4], bq[4];                    // B operands: row i's k, q
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                bk[s] = *reinterpret_cast<const half8*>(&Ks[i][32 * s + 8 * lq]);
                bq[s] = *reinterpret_cast<const half8*>(&Qs[i][32 * s + 8 * lq]);
            }
            for (int j = 0; j < 4; ++j) {
                half4 ha = {}, hp = {};
                if (j <= rt) {                     // wave-uniform
                    floatx4 ckk = {0.0f, 0.0f, 0.0f, 0.0f}, cqk = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        const half8 ak = *reinterpret_cast<const half8*>(&Ks[16 * j + lr][32 * s + 8 * lq]);
                        ckk = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak, bk[s], ckk, 0, 0, 0);
                        cqk = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak, bq[s], cqk, 0, 0, 0);
                    }
                    const float4 gj = *reinterpret_cast<const float4*>(&G.Gs[16 * j + 4 * lq]);
                    const float gjv[4] = {gj.x, gj.y, gj.z, gj.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int jj = 16 * j + 4 * lq + e;
                        const float dec = __builtin_amdgcn_exp2f(fminf(gi - gjv[e], 0.0f) * 1.4426950408889634f);
                        ha[e] = (_Float16)(jj < i ? -(bi * dec) * ckk[e] : 0.0f);
                        hp[e] = (_Float16)(jj <= i ? dec * cqk[e] : 0.0f);
                    }
                }
                *reinterpret_cast<half4*>(&Am[i][16 * j + 4 * lq]) = ha;
                *reinterpret_cast<half4*>(&Pm[i][16 * j + 4 * lq]) = hp;
            }

            // ---- 2. the diagonal block T_bb = (I + A_bb)^-1 of this wave's
            //      row tile b = rt, by substitution (lane m owns column m).
            //      The wave has just written that A tile itself (a wave's LDS
            //      accesses complete in order), so no workgroup barrier comes
            //      between.  Row i is v_i = e_i + sum_{j<i} (-A)_ij t_j,
            //      accumulated in order of j; written column by column (t_j,
            //      then its term in every later row), so the dependent chain
            //      is 16 steps long, not the 120 of the row-by-row order.
            if (lane < 16) {
                const int b0 = 16 * rt, m = lane;
                half8 ar[16][2];                   // rows 1..15 of -A_bb (columns 0-7, 8-15)
#pragma unroll
                for (int i2 = 1; i2 < 16; ++i2) {
                    ar[i2][0] = *reinterpret_cast<const half8*>(&Am[b0 + i2][b0]);
                    if (i2 > 8) ar[i2][1] = *reinterpret_cast<const half8*>(&Am[b0 + i2][b0 + 8]);
                }
                float v[16];
#pragma unroll
                for (int i2 = 0; i2 < 16; ++i2) v[i2] = (i2 == m) ? 1.0f : 0.0f;
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const float tj = v[j];
                    om = max_abs(om, tj);
                    Td[rt][j][m] = (_Float16)tj;
#pragma unroll
                    for (int i2 = j + 1; i2 < 16; ++i2) v[i2] += (float)ar[i2][j >> 3][j & 7] * tj;
                }
            }
        }
        __syncthreads();

        // ---- 3. [W | U~] by block forward substitution (16x16x16 f16)
        //      tiles: cc = 0,1 -> W k-col tiles 2w+cc; cc = 2,3 -> U~ v-col tiles 2w+cc-2
        floatx4 cu[4][2];
        half4 xh[4][4];                            // X_b fragments as f16 B operands
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const half4 tb = *reinterpret_cast<const half4*>(&Td[b][lr][4 * lq]);
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                const int col = 16 * (2 * w + (cc & 1)) + lr;
                floatx4 r;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int tk = 16 * b + 4 * lq + e;
                    // fma(h, s, 0) is the product, as one v_fma_mix_f32 that
                    // also widens the f16 operand
                    r[e] = cc < 2 ? __builtin_fmaf((float)Ks[tk][col], G.BG[tk], 0.0f)
                                  : __builtin_fmaf((float)Vs[tk][col], G.Bs[tk], 0.0f);
                }
#pragma unroll
                for (int k = 0; k < b; ++k) {
                    const half4 an = *reinterpret_cast<const half4*>(&Am[16 * b + lr][16 * k + 4 * lq]);
                    r = __builtin_amdgcn_mfma_f32_16x16x16f16(an, xh[k][cc], r, 0, 0, 0);
                }
                floatx4 x = {0.0f, 0.0f, 0.0f, 0.0f};
                x = __builtin_amdgcn_mfma_f32_16x16x16f16(tb, to_half4(r), x, 0, 0, 0);
                om = max_abs4(max_abs4(om, r), x);
                xh[b][cc] = to_half4(x);
                if (cc >= 2) cu[b][cc - 2] = x;
            }
        }

        // ---- 4. Q~ = diag(gamma) Q - P W and Y0 = P U~ (16x16x16 f16; the
        //      W / U~ fragments are the B operands as they stand)
        floatx4 cq[4][2], cy[4][2];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const int col = 16 * (2 * w + cc) + lr;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int tk = 16 * i + 4 * lq + e;
                    cq[i][cc][e] = __builtin_fmaf((float)Qs[tk][col], G.Eg[tk], 0.0f);
                }
                cy[i][cc] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        // -W fragments: the B operands of Q~ and, transposed, the -W output
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) xh[i][cc] = -xh[i][cc];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int kt = 0; kt <= i; ++kt) {
                const half4 ap = *reinterpret_cast<const half4*>(&Pm[16 * i + lr][16 * kt + 4 * lq]);
#pragma unroll
                for (int cc = 0; cc < 2; ++cc) {
                    cq[i][cc] = __builtin_amdgcn_mfma_f32_16x16x16f16(ap, xh[kt][cc], cq[i][cc], 0, 0, 0);
                    // Y0^T = U~^T P^T, transposed by swapping the operands: the
                    // U~ fragment as A and the P fragment as B (lane (r, q)
                    // then holds v-cols 16 vt + 4q .. +3 of token 16 i + r)
                    cy[i][cc] = __builtin_amdgcn_mfma_f32_16x16x16f16(xh[kt][cc + 2], ap, cy[i][cc], 0, 0, 0);
                }
            }
        }

#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) om = max_abs4(max_abs4(om, cq[i][cc]), cy[i][cc]);

        // ---- 5. outputs, all in the scan's fragment order (16-byte pieces;
        //      see the scan kernel for the piece layouts)
        // U~ and Y0^T: this wave's C fragments are the scan's fragments as
        // they stand (Y0^T is the accumulator layout of the scan's Y^T = S Q~^T)
        {
            const size_t base = hc * CHK * QM_DN_HD;
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const int vt = 2 * w + cc;
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    const size_t o = base + (size_t)((vt * 2 + p) * 64 + lane) * 8;
                    const half4 u0 = to_half4(cu[2 * p][cc]), u1 = to_half4(cu[2 * p + 1][cc]);
                    const half4 y0 = to_half4(cy[2 * p][cc]), y1 = to_half4(cy[2 * p + 1][cc]);
                    *reinterpret_cast<half8*>(A.Ut + o) = half8{u0[0], u0[1], u0[2], u0[3], u1[0], u1[1], u1[2], u1[3]};
                    *reinterpret_cast<half8*>(A.Y0t + o) = half8{y0[0], y0[1], y0[2], y0[3], y1[0], y1[1], y1[2], y1[3]};
                }
            }
        }
        // -W, Q~ and K~^T want four consecutive columns of one token (or
        // tokens of one column) per lane, the transpose of a C fragment.  A C
        // fragment read as an A operand is the transposed tile, so one
        // 16x16x16 product with an identity B operand transposes it in
        // registers (exactly: every product is x * 1 or x * 0 in fp32).
        half4 idm;                                // B[k][n] = (k == n): lane (n, kq) holds k = 4kq .. +3
#pragma unroll
        for (int e = 0; e < 4; ++e) idm[e] = (_Float16)(4 * lq + e == lr ? 1.0f : 0.0f);
        auto transpose = [&](half4 a) {
            return to_half4(__builtin_amdgcn_mfma_f32_16x16x16f16(a, idm, floatx4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0));
        };
        // -W and Q~: piece 4i + w holds col tiles 2w, 2w+1 of token block i
        {
            uint16_t* wdst = A.Wn + hc * CHK * QM_DN_HD;
            uint16_t* qdst = A.Qt + hc * CHK * QM_DN_HD;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const half4 w0 = transpose(xh[i][0]), w1 = transpose(xh[i][1]);
                const half4 q0 = transpose(to_half4(cq[i][0])), q1 = transpose(to_half4(cq[i][1]));
                const size_t o = (size_t)((4 * i + w) * 64 + lane) * 8;
                *reinterpret_cast<half8*>(wdst + o) = cat8(w0, w1);
                *reinterpret_cast<half8*>(qdst + o) = cat8(q0, q1);
            }
        }
        // K^T of the qk-head, once for both v-heads (the scan applies each
        // head's decays gamma_C / gamma_j to U instead): piece 2kt + p, kt =
        // 2w, 2w+1, holds token blocks 2p, 2p+1 of k-col tile kt; the A
        // operand of a K tile is a row read (token 16 tau + lr, cols 16 kt +
        // 4 lq .. +3)
        if (hh == 0) {
            uint16_t* dst = A.Ktt + ((size_t)qkh * A.nc + c) * CHK * QM_DN_HD;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int kt = 2 * w + t;
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    half4 hv[2];
#pragma unroll
                    for (int hb = 0; hb < 2; ++hb) {
                        const int tau = 2 * p + hb;
                        const half4 a = *reinterpret_cast<const half4*>(&Ks[16 * tau + lr][16 * kt + 4 * lq]);
                        hv[hb] = transpose(a);
                    }
                    *reinterpret_cast<half8*>(dst + (size_t)((2 * kt + p) * 64 + lane) * 8) = cat8(hv[0], hv[1]);
                }
            }
        }
        if (tid < CHK) A.Dt[hc * CHK + tid] = G.Kd[tid];
        if (tid == 0) A.gC[hc] = exp_fast(G.Gs[CHK - 1]);

        // ---- 6. precision guard statistics: each v channel's max |v| over
        //      the chunk, and +inf in channel 0 if an f16 operand would overflow
        if (!(om <= 65504.0f)) vbad[hh] = 1;
        __syncthreads();
        if (tid < QM_DN_HD) {
            float m = fmaxf(fmaxf(vred[hh][0][tid], vred[hh][1][tid]), fmaxf(vred[hh][2][tid], vred[hh][3][tid]));
            if (tid == 0 && vbad[hh]) m = __builtin_inff();
            A.vstat[((size_t)h * (A.nc + 1) + c) * QM_DN_HD + tid] = m;
        }
        if (c == 0) {
            // the entering state's row maxima (slot nc): two threads per row
            const int r = tid >> 1, half = tid & 1;
            const float* sp = A.state + (size_t)h * QM_DN_HEAD_ELEMS + (size_t)r * QM_DN_HD + 64 * half;
            float4 sv[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) sv[j] = ld4(sp + 4 * j);
            float m = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j)
                m = fmaxf(m, fmaxf(fmaxf(fabsf(sv[j].x), fabsf(sv[j].y)), fmaxf(fabsf(sv[j].z), fabsf(sv[j].w))));
            m = fmaxf(m, __shfl_xor(m, 1));
            if (half == 0) A.vstat[((size_t)h * (A.nc + 1) + A.nc) * QM_DN_HD + r] = m;
        }
    }
}

// ============================================================================
// Precision guard and the exact fallback
// ============================================================================
// The chunked path rounds its MFMA operands to f16 (11 bits).  That holds the
// bf16-path bar while a head's v rows (and state rows) are of comparable size;
// when a few rows are orders of magnitude larger than the rest, an output of
// a large row at a token where it happens to be small carries an absolute
// error of ~2^-11 of that row's scale, which the per-token RMSNorm then
// divides by the small rows' scale.  Such heads, heads whose magnitudes
// would approach f16's range, and any chunk whose f16 operands would
// overflow, take the exact path below instead: the reference's per-token
// recurrence in fp32.

// LDS of the exact path, one 64-token block at a time.
struct ExactLds {
    float qn[CHK][QM_DN_HD];                     // q: conv + SiLU, then normalised and scaled
    float kn[CHK][QM_DN_HD];                     // k: conv + SiLU, then normalised
    float vv[CHK][16];                           // this slice's v channels
    float4 gt[CHK];                              // alpha, beta, k^.q^, -
    float yb[CHK][16];                           // pre-norm outputs of the slice's rows
    float inv[2][CHK];                           // 1/||q||, 1/||k|| (1 where the norm is <= 1e-12)
};

// Whether head h takes the exact path.  A row's magnitude is its v
// channel's max |v| over the sequence or its entering state row's max,
// whichever is larger.  The f16 chunk operands give each row an error of
// ~2^-11 of its own scale, and the per-token RMSNorm divides it by the
// token's rms over the rows; that only exceeds the bf16 path's bar when a
// few rows dominate by orders of magnitude and can all be near zero at one
// token.  Measured on the chunked path (1024 tokens, decay 0.9999 per token,
// cold and warm states), with per-head output errors: 1 or 2 rows 128-256
// times the rest, 6.5e-3 to 2.5e-2; 4 to 16 such rows at up to 256 times,
// at most 4.8e-3; the synthetic 4B model's own layers (median row 15-124
// times below the largest), at most 4.5e-3.  So a head goes exact when
//   - its largest magnitude passes 2^11, or a chunk flagged an f16
//     overflow (+inf), or
//   - its median row lies more than 256 times below the largest, or
//   - its median row lies more than 64 times below the largest and fewer
//     than 4 rows are within 4 times of it.
// Uniform over the workgroup (every thread returns the same).
QM_DEV bool dn_guard_exact(const DnPrefillArgs& A, int h, float* red /* 264 floats */) {
    const int tid = threadIdx.x, lane = tid & 63, r = tid & 127, half = tid >> 7;
    const float* vs = A.vstat + (size_t)h * (A.nc + 1) * QM_DN_HD + r;
    float m = 0.0f;
#pragma unroll 8
    for (int c = half; c <= A.nc; c += 2) m = fmaxf(m, vs[(size_t)c * QM_DN_HD]);
    red[tid] = m;
    __syncthreads();
    const float mr = tid < 128 ? fmaxf(red[tid], red[tid + 128]) : 0.0f;
    const float wm = max_xor32(max_xor16(row_max16(mr)));
    if (lane == 0 && tid < 128) red[256 + (tid >> 6)] = wm;
    __syncthreads();
    const float mmax = fmaxf(red[256], red[257]);
    const uint64_t n256 = __ballot(tid < 128 && mr >= mmax * (1.0f / 256.0f));
    const uint64_t n64 = __ballot(tid < 128 && mr >= mmax * (1.0f / 64.0f));
    const uint64_t n4 = __ballot(tid < 128 && mr >= mmax * 0.25f);
    __syncthreads();
    if (lane == 0 && tid < 128) {
        red[258 + (tid >> 6)] = (float)__popcll(n256);
        red[260 + (tid >> 6)] = (float)__popcll(n64);
        red[262 + (tid >> 6)] = (float)__popcll(n4);
    }
    __syncthreads();
    const float c256 = red[258] + red[259], c64 = red[260] + red[261], c4 = red[262] + red[263];
    __syncthreads();                             // red may be reused
    return !(mmax <= 2048.0f) || c256 < 64.0f || (c64 < 64.0f && c4 < 4.0f);
}

// The exact path for one (v-head h, 16-row slice vt): gemv.rs:1119-1201 per
// token in fp32 on this slice's state rows, from the raw inputs (conv1d +
// SiLU, L2 norms, q scale and gates recomputed here, gemv.rs:1132-1172).
// The update is evaluated in one sweep over the old row,
//   p = alpha (S.k),  d = beta (v - p),  y = alpha (S.q) + d (k.q),
//   S <- alpha S + d k^T,
// which equals the reference's decay / retrieve / update / read order in
// real arithmetic.  Each 64-token block's outputs go to the slice's 4 KB of
// the (head, chunk) block of Yx as f32 [64 tokens][16 rows], where the out
// kernel normalises them; the final rows go to the state.
QM_DEV void dn_exact_rows(const DnPrefillArgs& A, int h, int vt, ExactLds& L) {
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int qkh = h >> 1;
    // recurrence: lane (rr, m) holds columns 8m .. 8m+7 of slice row rr
    const int rr = 4 * w + (lane >> 4), m = lane & 15;
    float* srow = A.state + (size_t)h * QM_DN_HEAD_ELEMS + (size_t)(16 * vt + rr) * QM_DN_HD + 8 * m;
    float sv[8];
    {
        const float4 a = ld4(srow), b = ld4(srow + 4);
        sv[0] = a.x; sv[1] = a.y; sv[2] = a.z; sv[3] = a.w;
        sv[4] = b.x; sv[5] = b.y; sv[6] = b.z; sv[7] = b.w;
    }
    const float ea = expf(A.a_log[h]), dtb = A.dt_bias[h];
    const float qscale = 1.0f / sqrtf((float)QM_DN_HD);
    // prep: thread (part, ci) owns q (part 0) or k (part 1) channel ci for
    // all tokens of a block; thread (vq, vr) owns v channel vr of the slice
    // for tokens 4vq .. 4vq+3
    const int part = tid >> 7, ci = tid & 127;
    const int chq = part * QM_DN_QK_DIM + qkh * QM_DN_HD + ci;
    const float4 wq = ld4(A.conv_w + (size_t)chq * 4);
    const int vr = tid & 15, vq = tid >> 4;
    const int chv = 2 * QM_DN_QK_DIM + h * QM_DN_HD + 16 * vt + vr;
    const float4 wv = ld4(A.conv_w + (size_t)chv * 4);
    float (*dst)[QM_DN_HD] = part ? L.kn : L.qn;
    // the three raw rows before the block (the conv buffer before token 0)
    float xp0 = A.conv_buf[(size_t)chq * 3], xp1 = A.conv_buf[(size_t)chq * 3 + 1];
    float xp2 = A.conv_buf[(size_t)chq * 3 + 2];

    for (int blk = 0; blk < A.nc; ++blk) {
        const int t0 = blk * CHK;
        const int nb = min(CHK, A.T - t0);
        // ---- q / k channel ci, 16 tokens per round of loads
#pragma unroll 1
        for (int g = 0; g < 4; ++g) {
            float xr[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int t = min(t0 + 16 * g + j, A.T - 1);
                xr[j] = bf16_to_f32(A.qkv[(size_t)t * QM_DN_QKV_DIM + chq]);
            }
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                dst[16 * g + j][ci] = silu_f(conv_taps4(xp0, xp1, xp2, xr[j], wq));
                xp0 = xp1; xp1 = xp2; xp2 = xr[j];
            }
        }
        // ---- v channel vr, tokens 4vq .. 4vq+3
        {
            float xv[7];
#pragma unroll
            for (int j = 0; j < 7; ++j) {
                const int t = t0 + 4 * vq - 3 + j;
                xv[j] = bf16_to_f32(A.qkv[(size_t)min(max(t, 0), A.T - 1) * QM_DN_QKV_DIM + chv]);
                if (t < 0) xv[j] = A.conv_buf[(size_t)chv * 3 + 3 + t];
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) L.vv[4 * vq + j][vr] = silu_f(conv_taps4(xv[j], xv[j + 1], xv[j + 2], xv[j + 3], wv));
        }
        __syncthreads();
        // ---- per token: gates (gemv.rs:1171-1172), L2 norms (:1151-1156)
        if (tid < CHK) {
            const int t = t0 + tid;
            float al = 1.0f, be = 0.0f;
            if (t < A.T) {
                al = expf(-ea * softplus_f(A.a[(size_t)t * QM_DN_V_HEADS + h] + dtb));
                be = 1.0f / (1.0f + expf(-A.b[(size_t)t * QM_DN_V_HEADS + h]));
            }
            float sq = 0.0f, sk = 0.0f, qk = 0.0f;
            for (int i = 0; i < QM_DN_HD; i += 4) {
                const float4 a = *reinterpret_cast<const float4*>(&L.qn[tid][i]);
                const float4 b = *reinterpret_cast<const float4*>(&L.kn[tid][i]);
                sq += a.x * a.x; sq += a.y * a.y; sq += a.z * a.z; sq += a.w * a.w;
                sk += b.x * b.x; sk += b.y * b.y; sk += b.z * b.z; sk += b.w * b.w;
                qk += a.x * b.x; qk += a.y * b.y; qk += a.z * b.z; qk += a.w * b.w;
            }
            const float nq = sqrtf(sq), nk = sqrtf(sk);
            const float iq = nq > 1e-12f ? 1.0f / nq : 1.0f, ik = nk > 1e-12f ? 1.0f / nk : 1.0f;
            L.inv[0][tid] = iq;
            L.inv[1][tid] = ik;
            L.gt[tid] = make_float4(al, be, qk * iq * ik * qscale, 0.0f);
        }
        __syncthreads();
        {
            const float* iv = L.inv[part];
#pragma unroll 8
            for (int j = 0; j < CHK; ++j) {
                float x = dst[j][ci] * iv[j];
                if (part == 0) x *= qscale;
                dst[j][ci] = x;
            }
        }
        __syncthreads();
        // ---- the recurrence over the block's tokens
#pragma unroll 2
        for (int j = 0; j < nb; ++j) {
            const float4 g = L.gt[j];
            const float4 k0 = *reinterpret_cast<const float4*>(&L.kn[j][8 * m]);
            const float4 k1 = *reinterpret_cast<const float4*>(&L.kn[j][8 * m + 4]);
            const float4 q0 = *reinterpret_cast<const float4*>(&L.qn[j][8 * m]);
            const float4 q1 = *reinterpret_cast<const float4*>(&L.qn[j][8 * m + 4]);
            const float v = L.vv[j][rr];
            const float kk[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
            const float qq[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
            float sk = 0.0f, sq = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                sk = fmaf(sv[e], kk[e], sk);
                sq = fmaf(sv[e], qq[e], sq);
            }
            sk = row_sum16(sk);
            sq = row_sum16(sq);
            const float dl = g.y * (v - g.x * sk);
            const float y = fmaf(g.x, sq, dl * g.z);
#pragma unroll
            for (int e = 0; e < 8; ++e) sv[e] = fmaf(dl, kk[e], g.x * sv[e]);
            if (m == 0) L.yb[j][rr] = y;
        }
        __syncthreads();
        {
            // f32 [64 tokens][16 rows] into the slice's 4 KB of block (h, blk)
            float* yo = reinterpret_cast<float*>(reinterpret_cast<char*>(A.Yx) +
                                                 ((size_t)h * A.nc + blk) * (QM_DN_HD * QM_DN_HD * 2) + 4096 * vt);
            st4(yo + 4 * tid, *reinterpret_cast<const float4*>(&L.yb[tid >> 2][4 * (tid & 3)]));
        }
        __syncthreads();
    }
    st4(srow, make_float4(sv[0], sv[1], sv[2], sv[3]));
    st4(srow + 4, make_float4(sv[4], sv[5], sv[6], sv[7]));
}

// ============================================================================
// 3. scan: sequential over chunks, one workgroup per (v-head, 16 state rows)
// ============================================================================
// Under the chunked delta rule every state row evolves on its own:
//   U_r = U~_r - W S_r^T,  S_r <- gamma_C S_r + (D U_r)^T K,
// D = diag(gamma_C / gamma), K the qk-head's keys (shared by its two v-heads)
// so a v-head's 128 rows split over 8 independent slices (grid 256).  The
// output Y_r = Y0_r + Q~ S_r^T of a chunk reads only its entry state, in the
// same f16 pieces the U product takes, so each wave forms its token tile of
// Y beside U, off the chain, and stores it in f16; the per-token norm over
// all 128 rows is left to the out kernel.
// S_r^T (k-cols x 16 rows, fp32) is held as eight C fragments; for k tile
// t, lane (r, q) = (lane & 15, lane >> 4) holds S[16 vt + r][16 t + 4q .. +3].
// All chunk operands arrive in fragment order as 16-byte pieces, piece
// (j, lane) at byte offset 16 (64 j + lane) of the (head, chunk) block:
//   -W, Q~   j = 4 i + p: tokens 16 i + (lane & 15), k-cols 32 p + 4 (lane >> 4)
//            + {0..3} (k step 2p) and + 16 + {0..3} (k step 2p+1);
//   K^T      j = 2 kt + p: k-col 16 kt + (lane & 15), tokens 32 p + 4 (lane >> 4)
//            + {0..3} and + 16 + {0..3} (per qk-head and chunk);
//   U~, Y0   j = 2 vt + p: row 16 vt + (lane & 15), tokens 32 p + 4 (lane >> 4)
//            + {0..3} and + 16 + {0..3}.
// A 16-byte piece is the A operand of one v_mfma_f32_16x16x32_f16: a product
// only needs A and B to agree on which k each (lane, element) holds, and the
// two C fragments of S^T k tiles 2p, 2p+1 (or of U token tiles 2p, 2p+1)
// concatenated hold exactly the k (token) set of piece p.
// A workgroup of four waves (one per SIMD) owns one (v-head, 16 rows) slice,
// so the per-chunk chain is split four ways: wave w forms U's token tile w
// (4 MFMAs) and Y's token tile w (4 MFMAs, same S pieces), and updates S^T
// k-tiles 2w, 2w+1 (4 MFMAs).  The f16 (D U) tiles and S pieces are exchanged
// through LDS, two barriers per chunk.
// Single buffers suffice: a wave writes Sx (Ux) only after passing the
// barrier that every wave reaches after its last read of the previous
// contents.  Each wave's chain operands for chunk c + 4 (Y's for c + 2)
// are loaded right after their last use in chunk c.
extern "C" __global__ __launch_bounds__(256) void qm_dn_prefill_scan(DnPrefillArgs A) {
    __shared__ half8 Sx[4][64];                  // S^T piece p (k-tiles 2p, 2p+1), f16
    __shared__ half4 Ux[4][64];                  // U token tile i, f16
    __shared__ ExactLds XL;                      // the exact path's block buffers
    __shared__ float gred[264];                  // guard reductions
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    // blocks are dealt to the 8 XCDs round-robin: keep a head's 8 row slices
    // on one XCD so its chunk operands are fetched into one L2
    // (XCD x takes v-heads 4x .. 4x+3, i.e. both v-heads of two qk-heads,
    // which read the same K^T pieces)
    const int b = blockIdx.x, xcd = b & 7, idx = b >> 3;
    const int h = 4 * xcd + (idx >> 3), vt = idx & 7;
    const int nc = A.nc;
    const size_t hbase = (size_t)h * nc, kbase = (size_t)(h >> 1) * nc;

    if (dn_guard_exact(A, h, gred)) {
        dn_exact_rows(A, h, vt, XL);
        if (tid == 0) A.mode[h * 8 + vt] = 1;
        return;
    }
    float om = 0.0f;                             // largest |U|, |S| converted to f16

    float* Srow = A.state + (size_t)h * QM_DN_HEAD_ELEMS + (size_t)(16 * vt + (lane & 15)) * QM_DN_HD + 4 * (lane >> 4);
    floatx4 S[2];                                // S^T k-tiles 2w, 2w+1 (fp32)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const float4 v = ld4(Srow + 16 * (2 * w + t));
        S[t] = floatx4{v.x, v.y, v.z, v.w};
    }

    auto blk = [&](const uint16_t* base, int c) {
        return base + (hbase + c) * (CHK * QM_DN_HD) + (size_t)lane * 8;
    };
    struct Ops {
        half8 w[4];                              // -W pieces 4w .. 4w+3 (token block w)
        half4 u;                                 // U~ token tile w
        half8 k[4];                              // K~^T pieces 4w .. 4w+3 (k-tiles 2w, 2w+1)
    };
    auto load_w = [&](Ops& o, int c) {
        const uint16_t* ws = blk(A.Wn, c) + 4 * w * 512;
#pragma unroll
        for (int p = 0; p < 4; ++p) o.w[p] = *reinterpret_cast<const half8*>(ws + p * 512);
    };
    auto load_u = [&](Ops& o, int c) {
        o.u = *reinterpret_cast<const half4*>(blk(A.Ut, c) + (2 * vt + (w >> 1)) * 512 + 4 * (w & 1));
    };
    auto load_k = [&](Ops& o, int c) {
        const uint16_t* ks = A.Ktt + (kbase + c) * (CHK * QM_DN_HD) + (size_t)lane * 8 + 4 * w * 512;
#pragma unroll
        for (int j = 0; j < 4; ++j) o.k[j] = *reinterpret_cast<const half8*>(ks + j * 512);
    };
    // Q~ pieces 4w .. 4w+3 (token block w) and the Y0^T tile w, two chunks ahead
    struct OpsY {
        half8 q[4];
        half4 y;
        float d;                                 // gamma_C / gamma_t of token 16 w + 4 (lane >> 4) + (lane & 3)
    };
    auto load_qy = [&](OpsY& o, int c) {
        const uint16_t* qs = blk(A.Qt, c) + 4 * w * 512;
#pragma unroll
        for (int p = 0; p < 4; ++p) o.q[p] = *reinterpret_cast<const half8*>(qs + p * 512);
        o.y = *reinterpret_cast<const half4*>(blk(A.Y0t, c) + (2 * vt + (w >> 1)) * 512 + 4 * (w & 1));
    };
    auto load_d = [&](OpsY& o, int c) {
        // one float per lane: a 256-byte load rather than a 16-byte one per
        // lane of 64 distinct bytes (the CU's load path bounds this kernel);
        // each lane's four tokens come from its quad by DPP
        o.d = A.Dt[(hbase + c) * CHK + 16 * w + 4 * (lane >> 4) + (lane & 3)];
    };
    // Y^T tile w of this slice: lane (r, q) holds rows 16 vt + 4 q .. +3 of
    // token 16 w + r.  The slice's outputs are stored token-major, [64
    // tokens][16 rows] f16 per (head, chunk, slice), so that this store is
    // 512 contiguous bytes per wave (a store scattered over 16 token rows of
    // 256 bytes cost the scan ~6 us: its memory path is what bounds it).
    auto y_store = [&](int c, half4 v) {
        *reinterpret_cast<half4*>(A.Yt + (((hbase + c) * 8 + vt) * CHK + 16 * w + (lane & 15)) * 16
                                  + 4 * (lane >> 4)) = v;
    };
    // gamma_C of 64 chunks at a time, one per lane (a vector load, so LDS
    // waits never wait on it), the next 64 fetched half way through
    auto load_g = [&](int c0) { return A.gC[hbase + min(c0 + lane, nc - 1)]; };
    float gv = load_g(0), gn = 0.0f;

    // One chunk: U tile w = U~ + (-W) S^T; Y^T tile w = Y0^T + S Q~^T (the
    // chunk's outputs, off the chain); exchange D U; S^T tiles <- gamma_C S^T
    // + K^T (D U); exchange S.
    // A wave's ~15 operand loads per chunk (1 KB each) take the CU's
    // address unit ~16 cycles apiece, ~960 cycles per chunk for the four
    // waves.  Each register set's next load is issued right after the
    // instruction that consumes it, so the loads drain while the wave waits
    // on MFMA and LDS latency (issued together after the state update they
    // held every wave ~700 cycles per chunk).
    auto step = [&](int c, Ops& o, OpsY& oy) {
        if ((c & 63) == 32) gn = load_g(c + 32);
        if ((c & 63) == 0 && c) gv = gn;
        const float g = readlane_f32(gv, c & 63);
        const int cn = min(c + 4, nc - 1), cy = min(c + 2, nc - 1);
        half8 sb[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) sb[p] = Sx[p][lane];
        floatx4 u0 = {(float)o.u[0], (float)o.u[1], (float)o.u[2], (float)o.u[3]};
        floatx4 u1 = {0.0f, 0.0f, 0.0f, 0.0f};
        __builtin_amdgcn_sched_barrier(0);
        load_u(o, cn);
        __builtin_amdgcn_sched_barrier(0);
        u0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.w[0], sb[0], u0, 0, 0, 0);
        u1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.w[1], sb[1], u1, 0, 0, 0);
        u0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.w[2], sb[2], u0, 0, 0, 0);
        u1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.w[3], sb[3], u1, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        load_w(o, cn);
        __builtin_amdgcn_sched_barrier(0);
        floatx4 y0 = {(float)oy.y[0], (float)oy.y[1], (float)oy.y[2], (float)oy.y[3]};
        floatx4 y1 = {0.0f, 0.0f, 0.0f, 0.0f};
        // Y^T = S Q~^T + Y0^T: the S piece as the A operand and the Q~ piece
        // as B (both hold the same k set per lane and register), so each
        // lane gets four consecutive rows of one token
        y0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(sb[0], oy.q[0], y0, 0, 0, 0);
        y1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(sb[1], oy.q[1], y1, 0, 0, 0);
        y0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(sb[2], oy.q[2], y0, 0, 0, 0);
        y1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(sb[3], oy.q[3], y1, 0, 0, 0);
        // U's rows (tokens) scaled by gamma_C / gamma_t: the S update
        // takes diag(gamma_C / gamma) U against the qk-head's K
        const floatx4 us = (u0 + u1) * floatx4{dpp_f32<0x00>(oy.d), dpp_f32<0x55>(oy.d),
                                               dpp_f32<0xAA>(oy.d), dpp_f32<0xFF>(oy.d)};
        Ux[w][lane] = to_half4(us);
        __builtin_amdgcn_sched_barrier(0);
        load_qy(oy, cy);
        load_d(oy, cy);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        // the range checks come after the barriers, off the chain's path
        om = max_abs4(om, us);
        half8 ub[2];
#pragma unroll
        for (int p = 0; p < 2; ++p) ub[p] = cat8(Ux[2 * p][lane], Ux[2 * p + 1][lane]);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            S[t] = S[t] * g;
#pragma unroll
            for (int p = 0; p < 2; ++p)
                S[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.k[2 * t + p], ub[p], S[t], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        load_k(o, cn);
        __builtin_amdgcn_sched_barrier(0);
        const half8 mine = cat8(to_half4(S[0]), to_half4(S[1]));
        Sx[w][lane] = mine;
        const floatx4 ys = y0 + y1;
        y_store(c, to_half4(ys));
        __syncthreads();
        om = max_abs4(max_abs4(max_abs4(om, S[0]), S[1]), ys);
    };

    // four chunks of the chain's operands and two of the outputs' operands
    // in flight (a wave has a SIMD to itself)
    Ops ops[4];
    OpsY opy[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        load_w(ops[i], min(i, nc - 1));
        load_u(ops[i], min(i, nc - 1));
        load_k(ops[i], min(i, nc - 1));
        if (i < 2) { load_qy(opy[i], min(i, nc - 1)); load_d(opy[i], min(i, nc - 1)); }
        __builtin_amdgcn_sched_barrier(0);
    }
    {
        const half8 mine = cat8(to_half4(S[0]), to_half4(S[1]));
        om = max_abs4(max_abs4(om, S[0]), S[1]);
        Sx[w][lane] = mine;
    }
    __syncthreads();
    int c = 0;
    for (; c + 3 < nc; c += 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) step(c + i, ops[i], opy[i & 1]);
    }
#pragma unroll
    for (int i = 0; i < 3; ++i)
        if (c + i < nc) step(c + i, ops[i], opy[i & 1]);
    // if an f16 copy of U or S overflowed, redo this slice exactly (the
    // entering state is still in place: the state is written only here)
    const float ow = max_xor32(max_xor16(row_max16(om)));
    if (lane == 0) gred[w] = ow;
    __syncthreads();
    if (!(fmaxf(fmaxf(gred[0], gred[1]), fmaxf(gred[2], gred[3])) <= 65504.0f)) {
        dn_exact_rows(A, h, vt, XL);
        if (tid == 0) A.mode[h * 8 + vt] = 1;
        return;
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) st4(Srow + 16 * (2 * w + t), make_float4(S[t][0], S[t][1], S[t][2], S[t][3]));
    if (tid == 0) A.mode[h * 8 + vt] = 0;
}

// ============================================================================
// 4. out: the gated RMSNorm (gemv.rs:1205-1219) of the scan's outputs, plus
//    the conv buffer update
// ============================================================================
// One workgroup per (chunk, v-head).  The head's 128 rows of Y for the
// chunk's 64 tokens come from the eight slices, each [64 tokens][16 rows],
// f16 (the scan stores Y^T fragments) or, for a slice that ran exactly,
// f32.  The norm runs 32 lanes per token with 4 consecutive values each, so
// z and the output move 512 contiguous bytes per token pair, with no
// staging through LDS.  At most 64 VGPRs, so that all of a 4096-token
// layer's 2048 workgroups (8 per CU) are resident at once.
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8)))
void qm_dn_prefill_out(DnPrefillArgs A) {
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int c = blockIdx.x / QM_DN_V_HEADS, h = blockIdx.x % QM_DN_V_HEADS;
    const size_t hc = (size_t)h * A.nc + c;

    if (c == 0) {
        // conv buffer after the prefill: the last three raw inputs (gemv.rs:1141-1146)
        const int ch = h * 256 + tid;
        float old[3] = {A.conv_buf[(size_t)ch * 3], A.conv_buf[(size_t)ch * 3 + 1], A.conv_buf[(size_t)ch * 3 + 2]};
        float nb[3];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int t = A.T - 3 + j;
            nb[j] = t >= 0 ? bf16_to_f32(A.qkv[(size_t)t * QM_DN_QKV_DIM + ch]) : old[A.T + j];
        }
#pragma unroll
        for (int j = 0; j < 3; ++j) A.conv_buf[(size_t)ch * 3 + j] = nb[j];
    }

    // Lane (col, token) = (8 (lane & 15), 16 w + (lane >> 4) + 4 q): rows
    // col .. col+7 of 4 tokens; z and the output are whole 256-byte token
    // rows per 16 lanes (16-byte accesses), and a token's 128 rows are one
    // DPP row, so the sum of squares is one row reduction.
    const int col = 8 * (lane & 15);
    const int tk0 = 16 * w + (lane >> 4);
    uint4 zr[4], yr[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int t = min(c * CHK + tk0 + 4 * q, A.T - 1);      // rows past T are not written
        zr[q] = *reinterpret_cast<const uint4*>(A.z + ((size_t)t * QM_DN_V_HEADS + h) * QM_DN_HD + col);
    }
    const uint16_t* ysrc = A.Yt + (hc * 8 + (col >> 4)) * (CHK * 16) + (col & 15);
#pragma unroll
    for (int q = 0; q < 4; ++q) yr[q] = *reinterpret_cast<const uint4*>(ysrc + (tk0 + 4 * q) * 16);
    // a slice the scan ran exactly has its rows as f32 [64 tokens][16 rows]
    // in its 4 KB of this (head, chunk) block instead
    const bool exl = A.mode[h * 8 + (col >> 4)] != 0;
    const float* xsrc = A.Yx + hc * (QM_DN_HD * QM_DN_HD / 2) + (col >> 4) * (CHK * 16) + (col & 15);
    const uint4 gw = *reinterpret_cast<const uint4*>(A.norm_w + col);
    const uint32_t gwv[4] = {gw.x, gw.y, gw.z, gw.w};
    float gg[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        gg[2 * e] = f16_to_f32((uint16_t)(gwv[e] & 0xffffu));
        gg[2 * e + 1] = f16_to_f32((uint16_t)(gwv[e] >> 16));
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t yv[4] = {yr[q].x, yr[q].y, yr[q].z, yr[q].w};
        float yq[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            yq[2 * e] = f16_to_f32((uint16_t)(yv[e] & 0xffffu));
            yq[2 * e + 1] = f16_to_f32((uint16_t)(yv[e] >> 16));
        }
        if (exl) {
            const float4 a = ld4(xsrc + (tk0 + 4 * q) * 16), b = ld4(xsrc + (tk0 + 4 * q) * 16 + 4);
            yq[0] = a.x; yq[1] = a.y; yq[2] = a.z; yq[3] = a.w;
            yq[4] = b.x; yq[5] = b.y; yq[6] = b.z; yq[7] = b.w;
        }
        float ss = yq[0] * yq[0];
#pragma unroll
        for (int e = 1; e < 8; ++e) ss = fmaf(yq[e], yq[e], ss);
        ss = row_sum16(ss);
        const int t = c * CHK + tk0 + 4 * q;
        if (t < A.T) {
            // 1/sqrt(mean + eps) as v_rsq_f32 (1 ulp), as the decode step
            // computes it; the exact sqrt and divide cost ~30 instructions
            const float inv_rms = __builtin_amdgcn_rsqf(ss * (1.0f / (float)QM_DN_HD) + 1e-6f);
            const uint32_t zv[4] = {zr[q].x, zr[q].y, zr[q].z, zr[q].w};
            uint32_t o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float z0 = bf16_to_f32((uint16_t)(zv[e] & 0xffffu)), z1 = bf16_to_f32((uint16_t)(zv[e] >> 16));
                o[e] = pack_bf16x2(yq[2 * e] * inv_rms * gg[2 * e] * silu_fast(z0),
                                   yq[2 * e + 1] * inv_rms * gg[2 * e + 1] * silu_fast(z1));
            }
            *reinterpret_cast<uint4*>(A.out + ((size_t)t * QM_DN_V_HEADS + h) * QM_DN_HD + col) =
                make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
}
