// gqa_prefill.hip -- full-attention GQA causal prefill for gfx950.
//
// Replaces the mixer slice of prefill_attn_layer (gemv.rs:1364-1444): per
// token QK RMSNorm (1+gamma) and partial RoPE at positions 0..S-1, the KV
// cache replaced by the normed/roped K and V (f16), causal softmax attention
// with kv head h/4, sigmoid output gate.
//
// qm_gqa_prefill_kv    K norm + RoPE -> f16 K cache; V -> f16 V cache and a
//                      transposed f16 copy V^T (keys contiguous per dim).
// qm_gqa_prefill_attn  flash attention on MFMA.  A workgroup owns 32 query
//                      tokens of all four query heads of one kv group (wave
//                      w = head 4g+w), so every K / V tile staged in LDS
//                      feeds four heads.  Scores are computed transposed,
//                      S^T = K Q^T (keys x rows), with v_mfma_f32_16x16x32:
//                      a lane of an S^T fragment then holds four consecutive
//                      keys of one row, which is exactly what the PV product
//                      (rows x dims, contracting keys) needs as its A operand
//                      once two 16-key fragments are paired; the V^T operand
//                      uses the same key pairing.  No lane shuffles between
//                      the two products.  Online softmax in base 2, fp32.
#include "qm_device.h"
#include "qm_kernel_args.h"
#include "qm_gqa_common.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

#define KT 64          // keys per tile
#define TQ 32          // query tokens per workgroup
#define KS_STRIDE 264  // f16 per K row in LDS (256 + 8 pad)
#define VT_STRIDE 72   // f16 per V^T row in LDS (64 + 8 pad)

QM_DEV float4 bf16x4_to_f32(uint2 u) {
    return make_float4(bf16_to_f32((uint16_t)(u.x & 0xffffu)), bf16_to_f32((uint16_t)(u.x >> 16)),
                       bf16_to_f32((uint16_t)(u.y & 0xffffu)), bf16_to_f32((uint16_t)(u.y >> 16)));
}

QM_DEV uint2 f32x4_to_f16(float4 x) {
    uint2 o;
    o.x = (uint32_t)f32_to_f16(x.x) | ((uint32_t)f32_to_f16(x.y) << 16);
    o.y = (uint32_t)f32_to_f16(x.z) | ((uint32_t)f32_to_f16(x.w) << 16);
    return o;
}

// ---------------------------------------------------------------------------
// K / V cache write (gemv.rs:1387-1400).  Workgroup = 64 tokens of kv head g.
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void qm_gqa_prefill_kv(GqaPrefillArgs A) {
    __shared__ _Float16 vs[64][264];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int g = blockIdx.x % QM_GQA_KV_HEADS;
    const int t0 = (blockIdx.x / QM_GQA_KV_HEADS) * 64;
    // K: wave w normalises and rotates tokens t0+16w .. t0+16w+15
    for (int j = 0; j < 16; ++j) {
        const int t = t0 + 16 * w + j;
        if (t >= A.S) break;                                     // wave-uniform
        const uint2 raw = *reinterpret_cast<const uint2*>(A.k + ((size_t)t * QM_GQA_KV_HEADS + g) * QM_GQA_HD + 4 * lane);
        const float4 x = norm_rope_head(bf16x4_to_f32(raw), A.k_norm, A.rope_cos + (size_t)t * 32,
                                        A.rope_sin + (size_t)t * 32, lane);
        *reinterpret_cast<uint2*>(A.k_cache + ((size_t)g * A.cap + t) * QM_GQA_HD + 4 * lane) = f32x4_to_f16(x);
    }
    // V: rows to the cache, and through LDS to V^T
    {
        const int i = tid >> 2, p = tid & 3, t = t0 + i;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            uint4 h16 = make_uint4(0, 0, 0, 0);
            if (t < A.S) {
                const uint4 raw = *reinterpret_cast<const uint4*>(A.v + ((size_t)t * QM_GQA_KV_HEADS + g) * QM_GQA_HD + 64 * p + 8 * q);
                const float4 lo = bf16x4_to_f32(make_uint2(raw.x, raw.y));
                const float4 hi = bf16x4_to_f32(make_uint2(raw.z, raw.w));
                const uint2 a = f32x4_to_f16(lo), b = f32x4_to_f16(hi);
                h16 = make_uint4(a.x, a.y, b.x, b.y);
                *reinterpret_cast<uint4*>(A.v_cache + ((size_t)g * A.cap + t) * QM_GQA_HD + 64 * p + 8 * q) = h16;
            }
            *reinterpret_cast<uint4*>(&vs[i][64 * p + 8 * q]) = h16;
        }
    }
    __syncthreads();
    {
        const int d = tid;
        uint16_t* dst = A.vt + ((size_t)g * QM_GQA_HD + d) * A.s_pad + t0;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            half8 hv;
#pragma unroll
            for (int e = 0; e < 8; ++e) hv[e] = vs[8 * q + e][d];
            *reinterpret_cast<half8*>(dst + 8 * q) = hv;
        }
    }
}

// ---------------------------------------------------------------------------
// Flash attention.  Lane (lr, lq) = (lane & 15, lane >> 4).
// ---------------------------------------------------------------------------
struct PrefillSmem {
    union {
        _Float16 qstage[4][TQ][KS_STRIDE];                 // q prep, per wave
        struct {
            _Float16 Ks[KT][KS_STRIDE];
            _Float16 Vts[QM_GQA_HD][VT_STRIDE];
        } kv;
    } u;
    float rowf[4][TQ];
};

extern "C" __global__ __launch_bounds__(256) void qm_gqa_prefill_attn(GqaPrefillArgs A) {
    __shared__ PrefillSmem sm;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, lq = lane >> 4;
    const int g = blockIdx.x % QM_GQA_KV_HEADS;
    const int nblk = A.s_pad / TQ;
    const int tb = nblk - 1 - (int)(blockIdx.x / QM_GQA_KV_HEADS);   // longest rows first
    const int t0 = tb * TQ;
    const int qh = 4 * g + w;

    // 1. q: RMSNorm (1+gamma) + RoPE at its position, f16, B fragments of S^T
    for (int j = 0; j < TQ; ++j) {
        const int t = t0 + j;
        float4 x = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (t < A.S) {                                              // wave-uniform
            const uint2 raw = *reinterpret_cast<const uint2*>(A.q_gate + ((size_t)t * QM_GQA_HEADS + qh) * (2 * QM_GQA_HD) + 4 * lane);
            x = norm_rope_head(bf16x4_to_f32(raw), A.q_norm, A.rope_cos + (size_t)t * 32,
                               A.rope_sin + (size_t)t * 32, lane);
        }
        *reinterpret_cast<uint2*>(&sm.u.qstage[w][j][4 * lane]) = f32x4_to_f16(x);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    half8 qf[2][8];                         // B[k = dim][n = row]: 8 dims of row n
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int s = 0; s < 8; ++s)
            qf[rt][s] = *reinterpret_cast<const half8*>(&sm.u.qstage[w][16 * rt + lr][32 * s + 8 * lq]);

    floatx4 O[2][16];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int dt = 0; dt < 16; ++dt) O[rt][dt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.0f, 0.0f};
    const float sl2 = (1.0f / 16.0f) * 1.4426950408889634f;     // 1/sqrt(256) * log2(e)

    const int nkt = (t0 + TQ + KT - 1) / KT;
    for (int kt = 0; kt < nkt; ++kt) {
        const int k0 = kt * KT;
        __syncthreads();                    // previous tile (or q staging) fully consumed
        // stage K tile [64 keys][256] and V^T tile [256 dims][64 keys]
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int piece = tid + 256 * r;                     // 2048 x 16 B each
            const int key = piece >> 5, col = 8 * (piece & 31);
            uint4 kv = make_uint4(0, 0, 0, 0);
            if (k0 + key < A.S)
                kv = *reinterpret_cast<const uint4*>(A.k_cache + ((size_t)g * A.cap + k0 + key) * QM_GQA_HD + col);
            *reinterpret_cast<uint4*>(&sm.u.kv.Ks[key][col]) = kv;
            const int d = piece >> 3, kc = 8 * (piece & 7);
            const uint4 vv = *reinterpret_cast<const uint4*>(A.vt + ((size_t)g * QM_GQA_HD + d) * A.s_pad + k0 + kc);
            *reinterpret_cast<uint4*>(&sm.u.kv.Vts[d][kc]) = vv;
        }
        __syncthreads();

        // S^T = K Q^T: fragment [kk][rt] holds keys k0+16kk+4lq+e of row 16rt+lr
        floatx4 sT[4][2];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            sT[kk][0] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
            sT[kk][1] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const half8 a = *reinterpret_cast<const half8*>(&sm.u.kv.Ks[16 * kk + lr][32 * s + 8 * lq]);
                sT[kk][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[0][s], sT[kk][0], 0, 0, 0);
                sT[kk][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[1][s], sT[kk][1], 0, 0, 0);
            }
        }
        // online softmax per row (base 2)
        half8 pf[2][2];
        float corr[2];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const int tok = t0 + 16 * rt + lr;
            float mx = -INFINITY;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int key = k0 + 16 * kk + 4 * lq + e;
                    const float s = key <= tok ? sT[kk][rt][e] * sl2 : -INFINITY;
                    sT[kk][rt][e] = s;
                    mx = fmaxf(mx, s);
                }
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float m_new = fmaxf(m_run[rt], mx);
            corr[rt] = (m_run[rt] == -INFINITY) ? 0.0f : exp2f(m_run[rt] - m_new);
            float ps = 0.0f;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float p = (m_new == -INFINITY) ? 0.0f : exp2f(sT[kk][rt][e] - m_new);
                    sT[kk][rt][e] = p;
                    ps += p;
                }
            ps += __shfl_xor(ps, 16);
            ps += __shfl_xor(ps, 32);
            l_run[rt] = l_run[rt] * corr[rt] + ps;
            m_run[rt] = m_new;
            // A operand of PV, k-step ks pairs key fragments 2ks and 2ks+1
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    pf[rt][ks][e] = (_Float16)sT[2 * ks][rt][e];
                    pf[rt][ks][4 + e] = (_Float16)sT[2 * ks + 1][rt][e];
                }
        }
        // rescale O: lane (dim lr, lq) holds rows 16rt + 4lq + e
        if (lq == 0) {
            sm.rowf[w][lr] = corr[0];
            sm.rowf[w][16 + lr] = corr[1];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const float4 f = *reinterpret_cast<const float4*>(&sm.rowf[w][16 * rt + 4 * lq]);
#pragma unroll
            for (int dt = 0; dt < 16; ++dt) {
                O[rt][dt][0] *= f.x; O[rt][dt][1] *= f.y; O[rt][dt][2] *= f.z; O[rt][dt][3] *= f.w;
            }
        }
        __builtin_amdgcn_wave_barrier();
        // O += P V   (16x16x32; B lane (dim, lq) holds keys 32ks+4lq+e and 32ks+16+4lq+e)
#pragma unroll
        for (int dt = 0; dt < 16; ++dt) {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const half4 v0 = *reinterpret_cast<const half4*>(&sm.u.kv.Vts[16 * dt + lr][32 * ks + 4 * lq]);
                const half4 v1 = *reinterpret_cast<const half4*>(&sm.u.kv.Vts[16 * dt + lr][32 * ks + 16 + 4 * lq]);
                half8 b;
                b[0] = v0[0]; b[1] = v0[1]; b[2] = v0[2]; b[3] = v0[3];
                b[4] = v1[0]; b[5] = v1[1]; b[6] = v1[2]; b[7] = v1[3];
                O[0][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pf[0][ks], b, O[0][dt], 0, 0, 0);
                O[1][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pf[1][ks], b, O[1][dt], 0, 0, 0);
            }
        }
    }

    // 3. out = (O / l) * sigmoid(gate), bf16 (gemv.rs:1441-1444)
    __builtin_amdgcn_wave_barrier();
    if (lq == 0) {
        sm.rowf[w][lr] = 1.0f / l_run[0];
        sm.rowf[w][16 + lr] = 1.0f / l_run[1];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
        const float4 inv = *reinterpret_cast<const float4*>(&sm.rowf[w][16 * rt + 4 * lq]);
        const float iv[4] = {inv.x, inv.y, inv.z, inv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = t0 + 16 * rt + 4 * lq + e;
            if (t >= A.S) continue;
            const uint16_t* gate = A.q_gate + ((size_t)t * QM_GQA_HEADS + qh) * (2 * QM_GQA_HD) + QM_GQA_HD;
            uint16_t* o = A.out + ((size_t)t * QM_GQA_HEADS + qh) * QM_GQA_HD;
#pragma unroll
            for (int dt = 0; dt < 16; ++dt) {
                const int d = 16 * dt + lr;
                const float gv = bf16_to_f32(gate[d]);
                o[d] = f32_to_bf16((O[rt][dt][e] * iv[e]) * sigmoid_f(gv));
            }
        }
    }
}
