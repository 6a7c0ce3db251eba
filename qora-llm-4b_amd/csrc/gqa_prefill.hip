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
//                      tokens of all four query heads of one kv group (8
//                      waves: head 4g + (w & 3), 16 rows each, two waves per
//                      SIMD), so every K / V tile staged in LDS feeds four
//                      heads.  Scores are computed transposed,
//                      S^T = K Q^T (keys x rows), with v_mfma_f32_16x16x32:
//                      a lane of an S^T fragment then holds four consecutive
//                      keys of one row, which is exactly what the PV product
//                      (rows x dims, contracting keys) needs as its A operand
//                      once two 16-key fragments are paired; the V^T operand
//                      uses the same key set per lane (the S^T rows are
//                      permuted so that set is 8 consecutive keys).  No lane
//                      shuffles between the two products.  Online softmax in
//                      base 2, fp32, with a lazily moved reference max.  K / V
//                      tiles are double-buffered in LDS and copied there by
//                      LDS DMA while the previous tile computes.
#include "qm_device.h"
#include "qm_kernel_args.h"
#include "qm_gqa_common.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

#define KT 64          // keys per tile
// Rows keep a reference max m and only move it when the tile max exceeds it
// by more than this (log2 units), so P = 2^(s - m) <= 2^8 stays exact enough
// in f16 and the O accumulators are rescaled only when a row's max jumps.
#define RESCALE_SLACK 8.0f
#define TQ 32          // query tokens per workgroup

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
// LDS (bytes): two tile buffers of 64 KB.  A buffer holds a 64-key tile in
// MFMA fragment order: 32 K blocks (kk, s) then 32 V^T blocks (dt, ks) of
// 1 KB, block entry l being the 16 bytes lane l reads for that product, so
// every fragment read is lane * 16 + an immediate (no bank conflicts, no
// per-read address registers).  The gather into that order is done by the
// per-lane source addresses of the LDS DMA.  The q staging area [8 waves]
// [16 rows][512 B] shares buffer 1 (consumed before tile 1 arrives), rows
// with their 16-byte chunks XOR swizzled (chunk c at c ^ swz_k(row)); then
// the per-wave row factors.
#define SM_BUF 65536
#define SM_V 32768
#define SM_ROWF (2 * SM_BUF)

// rows {b..b+3, b+8..b+11, b+16..b+19, b+24..b+27} (a read phase) -> distinct
// low 4 bits: bits 0,1 stay, bits 3,4 -> 2,3, bit 2 -> 4
QM_DEV int swz_k(int r) { return (r & 3) | (((r >> 3) & 3) << 2) | (((r >> 2) & 1) << 4); }

// Key held by row i of S^T fragment kk: the four fragments of a 64-key tile
// are arranged so that, for PV k-step ks = kk >> 1, a lane's pair of
// fragments 2ks, 2ks+1 holds the 8 consecutive keys 32 ks + 8 lq .. + 7.
QM_DEV int frag_key(int kk, int i) { return 32 * (kk >> 1) + 8 * (i >> 2) + 4 * (kk & 1) + (i & 3); }

// 16 bytes per lane from global memory straight into LDS: lane l writes
// lds + 16 l.  Issued as inline asm so that no compiler-inserted wait ties
// later LDS reads to it; completion is awaited explicitly (vmcnt) before the
// barrier that publishes the tile.  M0 has no other user in this kernel.
QM_DEV void dma16(const void* gsrc, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(gsrc), "s"(lds) : "memory", "m0");
}

extern "C" __global__ __launch_bounds__(512) void qm_gqa_prefill_attn(GqaPrefillArgs A) {
    __shared__ __attribute__((aligned(1024))) char sm[2 * SM_BUF + 8 * 16 * 4];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lq = lane >> 4;
    const int g = blockIdx.x % QM_GQA_KV_HEADS;
    const int nblk = A.s_pad / TQ;
    const int tb = nblk - 1 - (int)(blockIdx.x / QM_GQA_KV_HEADS);   // longest rows first
    const int t0 = tb * TQ;
    // wave w: query head 4g + (w & 3), rows r0 .. r0+15 of the block
    const int qh = 4 * g + (w & 3);
    const int r0 = t0 + 16 * (w >> 2);
    const int nkt = (t0 + TQ + KT - 1) / KT;
    const uint32_t sm_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)sm;
    float* rowf = reinterpret_cast<float*>(sm + SM_ROWF) + w * 16;

    // tile fetch: wave w moves K blocks 4w .. 4w+3 and V^T blocks 4w .. 4w+3
    const uint16_t* kbase = A.k_cache + (size_t)g * A.cap * QM_GQA_HD;
    const uint16_t* vbase = A.vt + (size_t)g * QM_GQA_HD * A.s_pad;
    auto fetch = [&](int kt, int buf) {
        const int k0 = kt * KT;
        const uint32_t kdst = sm_lds + buf * SM_BUF, vdst = kdst + SM_V;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int b = 4 * w + j, kk = b >> 3, s = b & 7;       // K block: S^T fragment kk, k-step s
            const int key = min(k0 + frag_key(kk, lr), A.S - 1);  // rows past S feed masked scores only
            dma16(kbase + (size_t)key * QM_GQA_HD + 32 * s + 8 * lq, kdst + 1024 * b);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int b = 4 * w + j, dt = b >> 1, ks = b & 1;      // V^T block: dims tile dt, keys step ks
            dma16(vbase + (size_t)(16 * dt + lr) * A.s_pad + k0 + 32 * ks + 8 * lq, vdst + 1024 * b);
        }
    };
    fetch(0, 0);                             // in flight during the q prep

    // 1. q: RMSNorm (1+gamma) + RoPE at its position, f16, staged in buffer 1
    char* qs = sm + SM_BUF + w * (16 * 512);
    for (int j = 0; j < 16; ++j) {
        const int t = r0 + j;
        float4 x = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (t < A.S) {                                              // wave-uniform
            const uint2 raw = *reinterpret_cast<const uint2*>(A.q_gate + ((size_t)t * QM_GQA_HEADS + qh) * (2 * QM_GQA_HD) + 4 * lane);
            x = norm_rope_head(bf16x4_to_f32(raw), A.q_norm, A.rope_cos + (size_t)t * 32,
                               A.rope_sin + (size_t)t * 32, lane);
        }
        *reinterpret_cast<uint2*>(qs + j * 512 + 16 * ((lane >> 1) ^ swz_k(j)) + 8 * (lane & 1)) = f32x4_to_f16(x);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    half8 qf[8];                            // B[k = dim][n = row]: 8 dims of row n
#pragma unroll
    for (int s = 0; s < 8; ++s)
        qf[s] = *reinterpret_cast<const half8*>(qs + lr * 512 + 16 * ((4 * s + lq) ^ swz_k(lr)));
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // tile 0 landed (this wave's part)
    __syncthreads();                        // tile 0 visible; q staging consumed

    floatx4 O[16];
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) O[dt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -INFINITY, l_run = 0.0f;
    const float sl2 = (1.0f / 16.0f) * 1.4426950408889634f;     // 1/sqrt(256) * log2(e)
    const int tok = r0 + lr;

    for (int kt = 0; kt < nkt; ++kt) {
        const int k0 = kt * KT, buf = kt & 1;
        // the other buffer was last read before the previous barrier
        if (kt + 1 < nkt) fetch(kt + 1, buf ^ 1);
        const char* Kb = sm + buf * SM_BUF;
        const char* Vb = Kb + SM_V;

        // S^T = K Q^T: fragment kk row i is key frag_key(kk, i) of the tile
        floatx4 sT[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            sT[kk] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const half8 a = *reinterpret_cast<const half8*>(Kb + (8 * kk + s) * 1024 + 16 * lane);
                sT[kk] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[s], sT[kk], 0, 0, 0);
            }
        }
        // online softmax per row (base 2); only tiles that reach past the
        // wave's first row need the causal mask
        const bool diag = k0 + KT - 1 > r0;
        float mx = -INFINITY;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float sc = sT[kk][e] * sl2;
                if (diag && k0 + frag_key(kk, 4 * lq + e) > tok) sc = -INFINITY;
                sT[kk][e] = sc;
                mx = fmaxf(mx, sc);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        // key 0 is visible to every row, so mx is finite from tile 0 on
        const float m_new = mx > m_run + RESCALE_SLACK ? mx : m_run;
        const float corr = __builtin_amdgcn_exp2f(m_run - m_new);    // 1 unless moved; 0 on tile 0
        float ps = 0.0f;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float pv = __builtin_amdgcn_exp2f(sT[kk][e] - m_new);
                sT[kk][e] = pv;
                ps += pv;
            }
        ps += __shfl_xor(ps, 16);
        ps += __shfl_xor(ps, 32);
        l_run = l_run * corr + ps;
        m_run = m_new;
        // A operand of PV k-step ks: keys 32 ks + 8 lq .. + 7 of row lr
        half8 pf[2];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                pf[ks][e] = (_Float16)sT[2 * ks][e];
                pf[ks][4 + e] = (_Float16)sT[2 * ks + 1][e];
            }
        // rescale O (lane (dim lr, lq) holds rows 4lq + e) when any row of
        // the wave moved its reference max
        if (__any(corr != 1.0f)) {
            if (lq == 0) rowf[lr] = corr;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const float4 f = *reinterpret_cast<const float4*>(&rowf[4 * lq]);
#pragma unroll
            for (int dt = 0; dt < 16; ++dt) {
                O[dt][0] *= f.x; O[dt][1] *= f.y; O[dt][2] *= f.z; O[dt][3] *= f.w;
            }
            __builtin_amdgcn_wave_barrier();
        }
        // O += P V   (16x16x32; B lane (dim, lq) holds keys 32 ks + 8 lq .. + 7)
#pragma unroll
        for (int dt = 0; dt < 16; ++dt)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const half8 b = *reinterpret_cast<const half8*>(Vb + (2 * dt + ks) * 1024 + 16 * lane);
                O[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pf[ks], b, O[dt], 0, 0, 0);
            }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // next tile landed (this wave's part)
        __syncthreads();                    // ... for every wave; this tile fully consumed
    }

    // 3. out = (O / l) * sigmoid(gate), bf16 (gemv.rs:1441-1444)
    if (lq == 0) rowf[lr] = 1.0f / l_run;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float4 inv = *reinterpret_cast<const float4*>(&rowf[4 * lq]);
    const float iv[4] = {inv.x, inv.y, inv.z, inv.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int t = r0 + 4 * lq + e;
        if (t >= A.S) continue;
        const uint16_t* gate = A.q_gate + ((size_t)t * QM_GQA_HEADS + qh) * (2 * QM_GQA_HD) + QM_GQA_HD;
        uint16_t* o = A.out + ((size_t)t * QM_GQA_HEADS + qh) * QM_GQA_HD;
#pragma unroll
        for (int dt = 0; dt < 16; ++dt) {
            const int d = 16 * dt + lr;
            const float gv = bf16_to_f32(gate[d]);
            o[d] = f32_to_bf16((O[dt][e] * iv[e]) * sigmoid_f(gv));
        }
    }
}
