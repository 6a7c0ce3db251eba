// gqa_decode.hip -- full-attention GQA decode step for gfx950.
//
// Replaces the mixer slice of forward_attn_decode (gemv.rs:927-1011):
// q/gate split, per-head RMSNorm (1+gamma) of q and k, partial RoPE on dims
// 0..63 at position pos, KV append (f16 cache), softmax attention over
// positions 0..pos with kv head h/4, sigmoid output gate.
//
// One launch per step: split-K flash decode.  Workgroup (b, g, split) owns
// `chunk` cache positions of kv head g and all four query heads of g, so
// each K/V byte is read from HBM once per step (the reference re-reads the
// cache once per query head, gemv.rs:963-986).  The last workgroup of a
// (b, g) to arrive merges the split partials and applies the gate.
//
// QK^T runs on MFMA (v_mfma_f32_16x16x32_f16).  q is fp32 in the reference,
// so it enters as an exact two-term f16 split q = q_hi + q_lo (rows 0..3 hi,
// rows 4..7 lo of the A operand); K comes straight from the f16 cache as the
// B operand and every product is exact in the fp32 accumulator.  PV stays on
// VALU: each lane owns 4 of the 256 dims of all four heads.
#include "qm_device.h"
#include "qm_kernel_args.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

#define GQA_PART_STRIDE 260   // acc[256], m, l, pad[2]

QM_DEV float ld_coherent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Per-head RMSNorm (1+gamma, eps 1e-6; gemv.rs:586-597) and split-half RoPE
// (gemv.rs:604-627) of one 256-wide head held by a wave: lane owns dims
// 4*lane..4*lane+3.  Lanes 0..7 hold dims 0..31, lanes 8..15 dims 32..63,
// so rotation partners are 8 lanes apart inside DPP row 0 (row_ror:8).
QM_DEV float4 norm_rope_head(float4 x, const uint16_t* gamma, const float* cos_row,
                             const float* sin_row, int lane) {
    float ss = x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
    ss = wave_sum64(ss);
    const float inv = 1.0f / sqrtf(ss / (float)QM_GQA_HD + 1e-6f);
    const uint2 gw = *reinterpret_cast<const uint2*>(gamma + 4 * lane);
    x.x = x.x * inv * (1.0f + f16_to_f32((uint16_t)(gw.x & 0xffffu)));
    x.y = x.y * inv * (1.0f + f16_to_f32((uint16_t)(gw.x >> 16)));
    x.z = x.z * inv * (1.0f + f16_to_f32((uint16_t)(gw.y & 0xffffu)));
    x.w = x.w * inv * (1.0f + f16_to_f32((uint16_t)(gw.y >> 16)));
    float4 pr;
    pr.x = dpp_f32<0x128>(x.x);
    pr.y = dpp_f32<0x128>(x.y);
    pr.z = dpp_f32<0x128>(x.z);
    pr.w = dpp_f32<0x128>(x.w);
    if (lane < 16) {
        const int i0 = (lane & 7) * 4;
        const float4 c = ld4(cos_row + i0), s = ld4(sin_row + i0);
        if (lane < 8) {          // x1 = own, x2 = partner: x1 c - x2 s
            x.x = x.x * c.x - pr.x * s.x; x.y = x.y * c.y - pr.y * s.y;
            x.z = x.z * c.z - pr.z * s.z; x.w = x.w * c.w - pr.w * s.w;
        } else {                 // x2 = own, x1 = partner: x2 c + x1 s
            x.x = x.x * c.x + pr.x * s.x; x.y = x.y * c.y + pr.y * s.y;
            x.z = x.z * c.z + pr.z * s.z; x.w = x.w * c.w + pr.w * s.w;
        }
    }
    return x;
}

extern "C" __global__ __launch_bounds__(256) void qm_gqa_decode(GqaDecodeArgs A) {
    __shared__ float qs[4][QM_GQA_HD];          // normed+roped q, heads 4g..4g+3
    __shared__ float wacc[4][4][QM_GQA_HD];     // per-wave partial PV
    __shared__ float wm[4][4], wl[4][4];
    __shared__ uint32_t is_last;

    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int bid = blockIdx.x;
    const int split = bid % A.nsplit;
    const int bg = bid / A.nsplit;
    const int g = bg % QM_GQA_KV_HEADS;
    const int b = bg / QM_GQA_KV_HEADS;
    int pos = A.pos ? A.pos[b] : A.max_pos;
    pos = pos < 0 ? 0 : (pos > A.max_pos ? A.max_pos : pos);
    const int L = pos + 1;
    const int t_begin = split * A.chunk;
    const int t_end = min(t_begin + A.chunk, L);

    const float* cos_row = A.rope_cos + (size_t)pos * (QM_GQA_ROT / 2);
    const float* sin_row = A.rope_sin + (size_t)pos * (QM_GQA_ROT / 2);
    const size_t kv_base = ((size_t)b * QM_GQA_KV_HEADS + g) * (size_t)A.cap * QM_GQA_HD;

    // 1. q prep: wave w handles query head 4g+w (gemv.rs:927-949).
    {
        const float* qg = A.q_gate + ((size_t)b * QM_GQA_HEADS + 4 * g + w) * (2 * QM_GQA_HD);
        float4 x = norm_rope_head(ld4(qg + 4 * lane), A.q_norm, cos_row, sin_row, lane);
        *reinterpret_cast<float4*>(&qs[w][4 * lane]) = x;
    }
    // 2. The split that holds position pos appends the new k, v (gemv.rs:946-956).
    if (t_begin <= pos && pos < t_end) {
        if (w == 0) {
            const float* kn = A.k_new + ((size_t)b * QM_GQA_KV_HEADS + g) * QM_GQA_HD;
            float4 x = norm_rope_head(ld4(kn + 4 * lane), A.k_norm, cos_row, sin_row, lane);
            uint2 o;
            o.x = (uint32_t)f32_to_f16(x.x) | ((uint32_t)f32_to_f16(x.y) << 16);
            o.y = (uint32_t)f32_to_f16(x.z) | ((uint32_t)f32_to_f16(x.w) << 16);
            *reinterpret_cast<uint2*>(A.k_cache + kv_base + (size_t)pos * QM_GQA_HD + 4 * lane) = o;
        } else if (w == 1) {
            const float* vn = A.v_new + ((size_t)b * QM_GQA_KV_HEADS + g) * QM_GQA_HD;
            float4 x = ld4(vn + 4 * lane);
            uint2 o;
            o.x = (uint32_t)f32_to_f16(x.x) | ((uint32_t)f32_to_f16(x.y) << 16);
            o.y = (uint32_t)f32_to_f16(x.z) | ((uint32_t)f32_to_f16(x.w) << 16);
            *reinterpret_cast<uint2*>(A.v_cache + kv_base + (size_t)pos * QM_GQA_HD + 4 * lane) = o;
        }
        __threadfence();
    }
    __syncthreads();
    __threadfence();

    // 3. A operand: row i (= lane & 15) is q_hi of head i (i < 4), q_lo of
    //    head i-4 (4 <= i < 8), zero otherwise.  K-step s, lane group
    //    aq = lane >> 4 and element e map to head dim 64*aq + 8*s + e; the B
    //    operand uses the same map, so lane group aq streams a contiguous
    //    128-byte quarter of each key row.
    const int arow = lane & 15, aq = lane >> 4;
    half8 afr[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float x = qs[arow & 3][64 * aq + 8 * s + e];
            const _Float16 hi = (_Float16)x;
            const _Float16 lo = (_Float16)(x - (float)hi);
            afr[s][e] = arow < 4 ? hi : (arow < 8 ? lo : (_Float16)0.0f);
        }
    }

    float m_run[4], l_run[4], acc[4][4];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        m_run[h] = -INFINITY; l_run[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[h][e] = 0.0f;
    }
    const float scale = 1.0f / sqrtf((float)QM_GQA_HD);

    // 4. Keys in rounds of 64: wave w takes keys base+16w .. base+16w+15.
    for (int base = t_begin; base < t_end; base += 64) {
        const int t0 = base + 16 * w;
        if (t0 >= t_end) break;
        const int tk = min(t0 + arow, t_end - 1);            // clamped: in bounds
        const uint16_t* krow = A.k_cache + kv_base + (size_t)tk * QM_GQA_HD + 64 * aq;
        half8 kf[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) kf[s] = *reinterpret_cast<const half8*>(krow + 8 * s);
        uint2 vr[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int tv = min(t0 + j, t_end - 1);
            vr[j] = *reinterpret_cast<const uint2*>(A.v_cache + kv_base + (size_t)tv * QM_GQA_HD + 4 * lane);
        }
        floatx4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 8; ++s) c = __builtin_amdgcn_mfma_f32_16x16x32_f16(afr[s], kf[s], c, 0, 0, 0);
        // D[i][j] sits in lane j + 16*(i/4), element i%4: lanes 0..15 carry
        // the hi rows, lanes 16..31 the lo rows of key j = lane & 15.
        const bool valid = (lane < 16) && (t0 + arow < t_end);
        float p[4];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const float sc = (c[h] + __shfl_xor(c[h], 16)) * scale;
            const float x = valid ? sc : -INFINITY;
            const float mt = readlane_f32(row_max16(x), 0);
            const float m_new = fmaxf(m_run[h], mt);
            const float corr = (m_run[h] == -INFINITY) ? 0.0f : expf(m_run[h] - m_new);
            p[h] = valid ? expf(sc - m_new) : 0.0f;
            const float ps = readlane_f32(row_sum16(p[h]), 0);
            l_run[h] = l_run[h] * corr + ps;
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[h][e] *= corr;
            m_run[h] = m_new;
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const float v0 = f16_to_f32((uint16_t)(vr[j].x & 0xffffu));
            const float v1 = f16_to_f32((uint16_t)(vr[j].x >> 16));
            const float v2 = f16_to_f32((uint16_t)(vr[j].y & 0xffffu));
            const float v3 = f16_to_f32((uint16_t)(vr[j].y >> 16));
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const float ph = readlane_f32(p[h], j);
                acc[h][0] = fmaf(ph, v0, acc[h][0]);
                acc[h][1] = fmaf(ph, v1, acc[h][1]);
                acc[h][2] = fmaf(ph, v2, acc[h][2]);
                acc[h][3] = fmaf(ph, v3, acc[h][3]);
            }
        }
    }

    // 5. Merge the four waves, write this split's partial.
    if (lane == 0) {
#pragma unroll
        for (int h = 0; h < 4; ++h) { wm[w][h] = m_run[h]; wl[w][h] = l_run[h]; }
    }
#pragma unroll
    for (int h = 0; h < 4; ++h)
        *reinterpret_cast<float4*>(&wacc[w][h][4 * lane]) = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
    __syncthreads();
    {
        const int h = w;                      // thread (h, lane): dims 4*lane..+3
        float M = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) M = fmaxf(M, wm[ww][h]);
        float Ls = 0.0f;
        float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) {
            const float f = (wm[ww][h] == -INFINITY) ? 0.0f : expf(wm[ww][h] - M);
            Ls += wl[ww][h] * f;
            const float4 a = *reinterpret_cast<const float4*>(&wacc[ww][h][4 * lane]);
            o.x += a.x * f; o.y += a.y * f; o.z += a.z * f; o.w += a.w * f;
        }
        float* P = A.partial + ((((size_t)b * QM_GQA_KV_HEADS + g) * A.nsplit + split) * 4 + h) * GQA_PART_STRIDE;
        st4(P + 4 * lane, o);
        if (lane == 0) { P[256] = M; P[257] = Ls; }
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = atomicAdd(&A.counters[b * QM_GQA_KV_HEADS + g], 1u);
        is_last = (prev == (uint32_t)A.nsplit - 1u) ? 1u : 0u;
    }
    __syncthreads();
    if (!is_last) return;
    __threadfence();

    // 6. Last arrival: merge splits in split order, gate, store.
    {
        const int h = w;
        float M = -INFINITY, Ls = 0.0f;
        float o0 = 0.0f, o1 = 0.0f, o2 = 0.0f, o3 = 0.0f;
        for (int s = 0; s < A.nsplit; ++s) {
            const float* P = A.partial + ((((size_t)b * QM_GQA_KV_HEADS + g) * A.nsplit + s) * 4 + h) * GQA_PART_STRIDE;
            const float ms = ld_coherent(P + 256);
            if (ms == -INFINITY) continue;
            const float ls = ld_coherent(P + 257);
            const float Mn = fmaxf(M, ms);
            const float fo = (M == -INFINITY) ? 0.0f : expf(M - Mn);
            const float fs = expf(ms - Mn);
            Ls = Ls * fo + ls * fs;
            o0 = o0 * fo + ld_coherent(P + 4 * lane + 0) * fs;
            o1 = o1 * fo + ld_coherent(P + 4 * lane + 1) * fs;
            o2 = o2 * fo + ld_coherent(P + 4 * lane + 2) * fs;
            o3 = o3 * fo + ld_coherent(P + 4 * lane + 3) * fs;
            M = Mn;
        }
        const float inv = 1.0f / Ls;
        const int qh = 4 * g + h;
        const float* gate = A.q_gate + ((size_t)b * QM_GQA_HEADS + qh) * (2 * QM_GQA_HD) + QM_GQA_HD + 4 * lane;
        const float4 gv = ld4(gate);
        float4 r;
        r.x = (o0 * inv) * sigmoid_f(gv.x);
        r.y = (o1 * inv) * sigmoid_f(gv.y);
        r.z = (o2 * inv) * sigmoid_f(gv.z);
        r.w = (o3 * inv) * sigmoid_f(gv.w);
        st4(A.out + ((size_t)b * QM_GQA_HEADS + qh) * QM_GQA_HD + 4 * lane, r);
        if (tid == 0)
            __hip_atomic_store(&A.counters[b * QM_GQA_KV_HEADS + g], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}
