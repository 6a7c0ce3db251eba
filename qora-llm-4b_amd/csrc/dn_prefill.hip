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
//   qm_dn_prefill_prep   conv1d + SiLU + L2 norm (+ q scale) + gates, one
//                        workgroup per (chunk, 128-channel head);
//   qm_dn_prefill_chunk  everything that does not depend on S0, fully
//                        parallel over (chunk, v-head): KK^T / QK^T on MFMA,
//                        T by blocked inversion in fp32 (16x16 diagonal
//                        blocks by substitution, off-diagonal blocks with
//                        fp32 MFMA), W, U~, Q~ = diag(gamma)Q - PW, Y0 = PU~
//                        on f16 MFMA;
//   qm_dn_prefill_scan   the sequential part, one workgroup per v-head with
//                        the 128x128 fp32 state in registers: three f16
//                        MFMA GEMMs per chunk plus the fused gated RMSNorm.
// The scan uses v_mfma_f32_16x16x16_f16 throughout because its fragment
// layouts chain without lane shuffles: the state's C fragment (4 consecutive
// k-cols per lane) is the B operand of U and Y, and U's C fragment (4
// consecutive tokens per lane) is the B operand of the state update.
#include "qm_device.h"
#include "qm_kernel_args.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

#define CHK QM_DN_CHUNK

QM_DEV half4 to_half4(floatx4 v) {
    half4 r;
    r[0] = (_Float16)v[0]; r[1] = (_Float16)v[1]; r[2] = (_Float16)v[2]; r[3] = (_Float16)v[3];
    return r;
}

// ============================================================================
// 1. prep: causal conv1d (gemv.rs:1132-1147), SiLU (:1149), per-head L2 norm
//    and q scale (:1151-1156), gates (:1171-1172).
// ============================================================================
extern "C" __global__ __launch_bounds__(256) void qm_dn_prefill_prep(DnPrefillArgs A) {
    __shared__ float act[CHK][129];
    const int tid = threadIdx.x;
    const int c = blockIdx.x / 64, gi = blockIdx.x % 64;     // 64 heads of 128 channels
    const int t0 = c * CHK;
    const int tpad = A.nc * CHK;
    const int chl = tid & 127, half = tid >> 7;
    const int ch = gi * 128 + chl;
    const float4 w = ld4(A.conv_w + ch * 4);
    const int tf = t0 + 32 * half;
    auto raw = [&](int t) -> float {
        if (t < 0) return A.conv_buf[(size_t)ch * 3 + 3 + t];   // buffer: x_{-3}, x_{-2}, x_{-1}
        if (t >= A.T) return 0.0f;
        return bf16_to_f32(A.qkv[(size_t)t * QM_DN_QKV_DIM + ch]);
    };
    float x3 = raw(tf - 3), x2 = raw(tf - 2), x1 = raw(tf - 1);
    for (int j = 0; j < 32; ++j) {
        const int t = tf + j;
        const float x0 = raw(t);
        float s = 0.0f;
        s = __fadd_rn(s, __fmul_rn(x3, w.x));
        s = __fadd_rn(s, __fmul_rn(x2, w.y));
        s = __fadd_rn(s, __fmul_rn(x1, w.z));
        s = __fadd_rn(s, __fmul_rn(x0, w.w));
        act[32 * half + j][chl] = (t < A.T) ? silu_f(s) : 0.0f;
        x3 = x2; x2 = x1; x1 = x0;
    }
    __syncthreads();

    const int tok = tid >> 2, part = tid & 3;                // 4 threads per token
    float v[32];
#pragma unroll
    for (int e = 0; e < 32; ++e) v[e] = act[tok][32 * part + e];
    uint16_t* dst;
    if (gi < 32) {
        // q (gi < 16) or k head: x /= ||x|| when ||x|| > 1e-12, q *= 1/sqrt(128)
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < 32; ++e) ss = fmaf(v[e], v[e], ss);
        ss += dpp_f32<0xB1>(ss);
        ss += dpp_f32<0x4E>(ss);
        const float norm = sqrtf(ss);
        const float inv = norm > 1e-12f ? 1.0f / norm : 1.0f;
        const float scale = gi < 16 ? 1.0f / sqrtf((float)QM_DN_HD) : 1.0f;
#pragma unroll
        for (int e = 0; e < 32; ++e) v[e] = (v[e] * inv) * scale;
        dst = (gi < 16 ? A.qh : A.kh) + ((size_t)(t0 + tok) * QM_DN_QK_HEADS + (gi & 15)) * QM_DN_HD + 32 * part;
    } else {
        dst = A.vv + ((size_t)(t0 + tok) * QM_DN_V_HEADS + (gi - 32)) * QM_DN_HD + 32 * part;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        half8 h;
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = (_Float16)v[8 * q + e];
        *reinterpret_cast<half8*>(dst + 8 * q) = h;
    }

    if (gi >= 32 && tid < 64) {
        // log alpha = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b);
        // padded tokens get alpha = 1, beta = 0 (no effect on the state).
        const int vh = gi - 32, t = t0 + tid;
        float g = 0.0f, be = 0.0f;
        if (t < A.T) {
            const float a_exp = expf(A.a_log[vh]);
            const float sp = softplus_f(A.a[(size_t)t * QM_DN_V_HEADS + vh] + A.dt_bias[vh]);
            g = -a_exp * sp;
            be = 1.0f / (1.0f + expf(-A.b[(size_t)t * QM_DN_V_HEADS + vh]));
        }
        // inclusive prefix sum over the chunk's 64 tokens (one wave)
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float o = __shfl_up(g, off);
            if (tid >= off) g += o;
        }
        A.G[(size_t)vh * tpad + t] = g;
        A.beta[(size_t)vh * tpad + t] = be;
    }
}

// ============================================================================
// 2. chunk: per (chunk, v-head), everything independent of the entering state
// ============================================================================
QM_DEV floatx4 mm16_f32(floatx4 c, const float (*X)[68], int xr, int xc, const float (*Y)[68], int yr,
                        int yc, int lane) {
    // c += X[xr:xr+16, xc:xc+16] * Y[yr:yr+16, yc:yc+16], fp32 MFMA 16x16x4
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const float a = X[xr + (lane & 15)][xc + 4 * ks + (lane >> 4)];
        const float b = Y[yr + 4 * ks + (lane >> 4)][yc + (lane & 15)];
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    }
    return c;
}

QM_DEV void store_c16(float (*D)[68], int r0, int c0, floatx4 c, float sgn, int lane) {
#pragma unroll
    for (int e = 0; e < 4; ++e) D[r0 + 4 * (lane >> 4) + e][c0 + (lane & 15)] = sgn * c[e];
}

extern "C" __global__ __launch_bounds__(256) void qm_dn_prefill_chunk(DnPrefillArgs A) {
    __shared__ _Float16 Ks[CHK][136];
    __shared__ _Float16 Qs[CHK][136];
    __shared__ _Float16 Kt[QM_DN_HD][72];
    __shared__ _Float16 Vt[QM_DN_HD][72];
    __shared__ _Float16 Pm[CHK][72];
    __shared__ float Af[CHK][68];
    __shared__ float Tf[CHK][68];
    __shared__ float scr[4][16][68];
    __shared__ float Gs[CHK], Bs[CHK], Eg[CHK], BG[CHK], Kd[CHK];

    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int c = blockIdx.x / QM_DN_V_HEADS, h = blockIdx.x % QM_DN_V_HEADS;
    const int qkh = h >> 1;
    const int t0 = c * CHK;
    const int tpad = A.nc * CHK;
    const size_t hc = (size_t)h * A.nc + c;
    const int lr = lane & 15, lq = lane >> 4;

    // ---- 0. load K, Q (row-major and K, V transposed) and the gates
    {
        const int i = tid >> 2, p = tid & 3;
        const uint16_t* kr = A.kh + ((size_t)(t0 + i) * QM_DN_QK_HEADS + qkh) * QM_DN_HD + 32 * p;
        const uint16_t* qr = A.qh + ((size_t)(t0 + i) * QM_DN_QK_HEADS + qkh) * QM_DN_HD + 32 * p;
        const uint16_t* vr = A.vv + ((size_t)(t0 + i) * QM_DN_V_HEADS + h) * QM_DN_HD + 32 * p;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const half8 kv = *reinterpret_cast<const half8*>(kr + 8 * q);
            const half8 qv = *reinterpret_cast<const half8*>(qr + 8 * q);
            const half8 vv = *reinterpret_cast<const half8*>(vr + 8 * q);
            *reinterpret_cast<half8*>(&Ks[i][32 * p + 8 * q]) = kv;
            *reinterpret_cast<half8*>(&Qs[i][32 * p + 8 * q]) = qv;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                Kt[32 * p + 8 * q + e][i] = kv[e];
                Vt[32 * p + 8 * q + e][i] = vv[e];
            }
        }
        if (tid < CHK) {
            Gs[tid] = A.G[(size_t)h * tpad + t0 + tid];
            Bs[tid] = A.beta[(size_t)h * tpad + t0 + tid];
        }
        // T: zero the blocks above the block diagonal
        for (int idx = tid; idx < 6 * 256; idx += 256) {
            const int blk = idx >> 8, e = idx & 255;
            const int rb = blk < 3 ? 0 : (blk < 5 ? 1 : 2);
            const int cb = blk < 3 ? blk + 1 : (blk < 5 ? blk - 1 : 3);
            Tf[16 * rb + (e >> 4)][16 * cb + (e & 15)] = 0.0f;
        }
    }
    __syncthreads();
    if (tid < CHK) {
        Eg[tid] = expf(Gs[tid]);                  // gamma_i
        BG[tid] = Bs[tid] * Eg[tid];              // beta_i gamma_i
        Kd[tid] = expf(Gs[CHK - 1] - Gs[tid]);    // gamma_C / gamma_i
    }

    // ---- 1. KK^T and QK^T (16x16x32 f16), masked and decayed
    {
        const int i0 = 16 * w;
        for (int j = 0; j <= w; ++j) {
            floatx4 ckk = {0.0f, 0.0f, 0.0f, 0.0f}, cqk = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int kk = 32 * s + 8 * lq;
                const half8 ak = *reinterpret_cast<const half8*>(&Ks[i0 + lr][kk]);
                const half8 aq = *reinterpret_cast<const half8*>(&Qs[i0 + lr][kk]);
                const half8 bk = *reinterpret_cast<const half8*>(&Ks[16 * j + lr][kk]);
                ckk = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak, bk, ckk, 0, 0, 0);
                cqk = __builtin_amdgcn_mfma_f32_16x16x32_f16(aq, bk, cqk, 0, 0, 0);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int i = i0 + 4 * lq + e, jj = 16 * j + lr;
                const float dec = jj <= i ? expf(Gs[i] - Gs[jj]) : 0.0f;
                Af[i][jj] = jj < i ? Bs[i] * dec * ckk[e] : 0.0f;
                Pm[i][jj] = (_Float16)(jj <= i ? dec * cqk[e] : 0.0f);
            }
        }
        for (int j = w + 1; j < 4; ++j) {
#pragma unroll
            for (int e = 0; e < 4; ++e) Pm[i0 + 4 * lq + e][16 * j + lr] = (_Float16)0.0f;
        }
    }
    __syncthreads();

    // ---- 2. T = (I + A)^-1
    // 2a. diagonal 16x16 blocks by forward substitution (lane m owns column m)
    if (lane < 16) {
        const int b0 = 16 * w, m = lane;
        float t[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float v = (i == m) ? 1.0f : 0.0f;
#pragma unroll
            for (int j = 0; j < i; ++j) v -= Af[b0 + i][b0 + j] * t[j];
            t[i] = v;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) Tf[b0 + i][b0 + m] = t[i];
    }
    __syncthreads();
    // 2b. T_{2p+1,2p} = -T_{2p+1,2p+1} A_{2p+1,2p} T_{2p,2p}
    if (w < 2) {
        const int r = 16 * (2 * w + 1), cb = 16 * (2 * w);
        floatx4 m = {0.0f, 0.0f, 0.0f, 0.0f};
        m = mm16_f32(m, Af, r, cb, Tf, cb, cb, lane);
        store_c16(scr[w], 0, 0, m, 1.0f, lane);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        floatx4 t = {0.0f, 0.0f, 0.0f, 0.0f};
        t = mm16_f32(t, Tf, r, r, scr[w], 0, 0, lane);
        store_c16(Tf, r, cb, t, -1.0f, lane);
    }
    __syncthreads();
    // 2c. lower-left 32x32 quadrant: T21 = -T22 (A21 T11) with 2x2 blocks
    {
        const int rb = 2 + (w >> 1), cb = w & 1;
        floatx4 m = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int kb = cb; kb < 2; ++kb) m = mm16_f32(m, Af, 16 * rb, 16 * kb, Tf, 16 * kb, 16 * cb, lane);
        store_c16(scr[w], 0, 0, m, 1.0f, lane);
    }
    __syncthreads();
    {
        const int rb = 2 + (w >> 1), cb = w & 1;
        floatx4 t = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int kb = 2; kb <= rb; ++kb) t = mm16_f32(t, Tf, 16 * rb, 16 * kb, scr[(kb - 2) * 2 + cb], 0, 0, lane);
        __syncthreads();   // every wave has read T_{3,2} (rb == 3) before any block is written
        store_c16(Tf, 16 * rb, 16 * cb, t, -1.0f, lane);
    }
    __syncthreads();

    // ---- 3. W = T diag(beta gamma) K and U~ = T diag(beta) V (16x16x32 f16)
    //      wave w owns k-col tiles 2w, 2w+1 of W and v-col tiles 2w, 2w+1 of U~
    floatx4 cw[4][2], cu[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            cw[i][cc] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
            cu[i][cc] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int s = 0; s <= (i >> 1); ++s) {
            const int row = 16 * i + lr, k0 = 32 * s + 8 * lq;
            half8 a1, a2;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float tv = Tf[row][k0 + e];
                a1[e] = (_Float16)(tv * BG[k0 + e]);
                a2[e] = (_Float16)(tv * Bs[k0 + e]);
            }
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const int col = 16 * (2 * w + cc) + lr;
                const half8 bk = *reinterpret_cast<const half8*>(&Kt[col][k0]);
                const half8 bv = *reinterpret_cast<const half8*>(&Vt[col][k0]);
                cw[i][cc] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bk, cw[i][cc], 0, 0, 0);
                cu[i][cc] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2, bv, cu[i][cc], 0, 0, 0);
            }
        }
    }

    // ---- 4. Q~ = diag(gamma) Q - P W and Y0 = P U~ (16x16x16 f16; the W / U~
    //      C fragments are the B operands as they stand)
    floatx4 cq[4][2], cy[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const int col = 16 * (2 * w + cc) + lr;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int tk = 16 * i + 4 * lq + e;
                cq[i][cc][e] = Eg[tk] * (float)Qs[tk][col];
            }
            cy[i][cc] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int kt = 0; kt <= i; ++kt) {
            const half4 ap = *reinterpret_cast<const half4*>(&Pm[16 * i + lr][16 * kt + 4 * lq]);
            const half4 an = -ap;
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                cq[i][cc] = __builtin_amdgcn_mfma_f32_16x16x16f16(an, to_half4(cw[kt][cc]), cq[i][cc], 0, 0, 0);
                cy[i][cc] = __builtin_amdgcn_mfma_f32_16x16x16f16(ap, to_half4(cu[kt][cc]), cy[i][cc], 0, 0, 0);
            }
        }
    }

    // ---- 5. outputs
    // U~^T and Y0^T: lane holds 4 consecutive tokens of one v-row -> 8-byte stores
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const int row = 16 * (2 * w + cc) + lr;
            const size_t o = (hc * QM_DN_HD + row) * CHK + 16 * i + 4 * lq;
            *reinterpret_cast<half4*>(A.Ut + o) = to_half4(cu[i][cc]);
            *reinterpret_cast<half4*>(A.Y0t + o) = to_half4(cy[i][cc]);
        }
    // K~^T = (gamma_C / gamma_j) K^T
    {
        const int row = tid >> 1, p = tid & 1;
        uint16_t* dst = A.Ktt + (hc * QM_DN_HD + row) * CHK + 32 * p;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            half8 hv;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int tk = 32 * p + 8 * q + e;
                hv[e] = (_Float16)((float)Kt[row][tk] * Kd[tk]);
            }
            *reinterpret_cast<half8*>(dst + 8 * q) = hv;
        }
    }
    if (tid == 0) A.gC[hc] = expf(Gs[CHK - 1]);
    __syncthreads();     // Ks / Qs are free: stage -W and Q~ token-major
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const int col = 16 * (2 * w + cc) + lr;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int tk = 16 * i + 4 * lq + e;
                Ks[tk][col] = (_Float16)(-cw[i][cc][e]);
                Qs[tk][col] = (_Float16)cq[i][cc][e];
            }
        }
    __syncthreads();
    {
        uint16_t* wdst = A.Wn + hc * CHK * QM_DN_HD;
        uint16_t* qdst = A.Qt + hc * CHK * QM_DN_HD;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int piece = tid + 256 * r;          // 1024 pieces of 8 halfs
            const int row = piece >> 4, col = 8 * (piece & 15);
            *reinterpret_cast<half8*>(wdst + row * QM_DN_HD + col) = *reinterpret_cast<const half8*>(&Ks[row][col]);
            *reinterpret_cast<half8*>(qdst + row * QM_DN_HD + col) = *reinterpret_cast<const half8*>(&Qs[row][col]);
        }
    }
}

// ============================================================================
// 3. scan: per v-head, sequential over chunks, state in registers
// ============================================================================
// Wave w owns state rows 16w..16w+15; for k-col tile t the lane (r, q) =
// (lane & 15, lane >> 4) holds S[16w + r][16t + 4q .. 16t + 4q + 3].
extern "C" __global__ __launch_bounds__(512) void qm_dn_prefill_scan(DnPrefillArgs A) {
    __shared__ _Float16 Wb[CHK][136];
    __shared__ _Float16 Qb[CHK][136];
    __shared__ _Float16 Kb[QM_DN_HD][72];
    __shared__ float ys[CHK][132];

    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, lq = lane >> 4;
    const int h = blockIdx.x;

    // conv buffer after the prefill: the last three raw inputs (gemv.rs:1141-1146)
    {
        const int ch = h * 512 + tid;
        if (ch < QM_DN_QKV_DIM) {
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
    }

    float* Sg = A.state + (size_t)h * QM_DN_HEAD_ELEMS;
    floatx4 S[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const float4 v = ld4(Sg + (size_t)(16 * w + lr) * QM_DN_HD + 16 * t + 4 * lq);
        S[t] = floatx4{v.x, v.y, v.z, v.w};
    }

    // per-chunk operand pieces of this thread: 2 of -W, 2 of Q~, 2 of K~^T
    // (16 bytes each), and this wave's U~^T / Y0^T fragments
    half8 pw[2], pq[2], pk[2];
    half4 pu[4], py[4];
    auto fetch = [&](int c) {
        const size_t hc = (size_t)h * A.nc + c;
        const uint16_t* wsrc = A.Wn + hc * CHK * QM_DN_HD;
        const uint16_t* qsrc = A.Qt + hc * CHK * QM_DN_HD;
        const uint16_t* ksrc = A.Ktt + hc * QM_DN_HD * CHK;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int piece = tid + 512 * r;
            pw[r] = *reinterpret_cast<const half8*>(wsrc + 8 * piece);
            pq[r] = *reinterpret_cast<const half8*>(qsrc + 8 * piece);
            pk[r] = *reinterpret_cast<const half8*>(ksrc + 8 * piece);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const size_t o = (hc * QM_DN_HD + 16 * w + lr) * CHK + 16 * i + 4 * lq;
            pu[i] = *reinterpret_cast<const half4*>(A.Ut + o);
            py[i] = *reinterpret_cast<const half4*>(A.Y0t + o);
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int piece = tid + 512 * r;
            *reinterpret_cast<half8*>(&Wb[piece >> 4][8 * (piece & 15)]) = pw[r];
            *reinterpret_cast<half8*>(&Qb[piece >> 4][8 * (piece & 15)]) = pq[r];
            *reinterpret_cast<half8*>(&Kb[piece >> 3][8 * (piece & 7)]) = pk[r];
        }
    };

    fetch(0);
    stage();
    __syncthreads();
    const uint16_t* zbase = A.z;
    for (int c = 0; c < A.nc; ++c) {
        half4 cu_h[4];
        floatx4 uu[4], yy[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uu[i] = floatx4{(float)pu[i][0], (float)pu[i][1], (float)pu[i][2], (float)pu[i][3]};
            yy[i] = floatx4{(float)py[i][0], (float)py[i][1], (float)py[i][2], (float)py[i][3]};
        }
        const float gC = A.gC[(size_t)h * A.nc + c];
        if (c + 1 < A.nc) fetch(c + 1);
        half4 sh[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) sh[t] = to_half4(S[t]);
        // U = U~ - W S^T, Y = Y0 + Q~ S^T   (tokens x rows, K = k-cols)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const half4 aw = *reinterpret_cast<const half4*>(&Wb[16 * i + lr][16 * t + 4 * lq]);
                const half4 aq = *reinterpret_cast<const half4*>(&Qb[16 * i + lr][16 * t + 4 * lq]);
                uu[i] = __builtin_amdgcn_mfma_f32_16x16x16f16(aw, sh[t], uu[i], 0, 0, 0);
                yy[i] = __builtin_amdgcn_mfma_f32_16x16x16f16(aq, sh[t], yy[i], 0, 0, 0);
            }
            cu_h[i] = to_half4(uu[i]);
#pragma unroll
            for (int e = 0; e < 4; ++e) ys[16 * i + 4 * lq + e][16 * w + lr] = yy[i][e];
        }
        // S^T <- gamma_C S^T + K~^T U   (k-cols x rows, K = tokens)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            S[t] = S[t] * gC;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const half4 ak = *reinterpret_cast<const half4*>(&Kb[16 * t + lr][16 * i + 4 * lq]);
                S[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(ak, cu_h[i], S[t], 0, 0, 0);
            }
        }
        __syncthreads();
        // gated RMSNorm (gemv.rs:1205-1219): thread (token, part) owns rows
        // 16*part .. 16*part+15 of one token; 8 lanes per token.
        {
            const int tk = tid >> 3, part = tid & 7;
            const int t = c * CHK + tk;
            float y[16];
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                y[e] = ys[tk][16 * part + e];
                ss = fmaf(y[e], y[e], ss);
            }
            ss += dpp_f32<0xB1>(ss);
            ss += dpp_f32<0x4E>(ss);
            ss += dpp_f32<0x141>(ss);
            if (t < A.T) {
                const float inv_rms = 1.0f / sqrtf(ss / (float)QM_DN_HD + 1e-6f);
                const size_t off = ((size_t)t * QM_DN_V_HEADS + h) * QM_DN_HD + 16 * part;
                const half8 z0 = *reinterpret_cast<const half8*>(zbase + off);   // raw bits, bf16
                const half8 z1 = *reinterpret_cast<const half8*>(zbase + off + 8);
                uint16_t ob[16];
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const uint16_t zb = __builtin_bit_cast(uint16_t, e < 8 ? z0[e] : z1[e - 8]);
                    const float zz = bf16_to_f32(zb);
                    const float gm = f16_to_f32(A.norm_w[16 * part + e]);
                    ob[e] = f32_to_bf16(y[e] * inv_rms * gm * silu_f(zz));
                }
                uint4 o0, o1;
                o0.x = ob[0] | ((uint32_t)ob[1] << 16); o0.y = ob[2] | ((uint32_t)ob[3] << 16);
                o0.z = ob[4] | ((uint32_t)ob[5] << 16); o0.w = ob[6] | ((uint32_t)ob[7] << 16);
                o1.x = ob[8] | ((uint32_t)ob[9] << 16); o1.y = ob[10] | ((uint32_t)ob[11] << 16);
                o1.z = ob[12] | ((uint32_t)ob[13] << 16); o1.w = ob[14] | ((uint32_t)ob[15] << 16);
                *reinterpret_cast<uint4*>(A.out + off) = o0;
                *reinterpret_cast<uint4*>(A.out + off + 8) = o1;
            }
        }
        if (c + 1 < A.nc) stage();
        __syncthreads();
    }
#pragma unroll
    for (int t = 0; t < 8; ++t)
        st4(Sg + (size_t)(16 * w + lr) * QM_DN_HD + 16 * t + 4 * lq, make_float4(S[t][0], S[t][1], S[t][2], S[t][3]));
}
