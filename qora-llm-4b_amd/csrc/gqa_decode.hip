// gqa_decode.hip -- full-attention GQA decode step for gfx950.
//
// Replaces the mixer slice of forward_attn_decode (gemv.rs:927-1011):
// q/gate split, per-head RMSNorm (1+gamma) of q and k, partial RoPE on dims
// 0..63 at position pos, KV append (f16 cache), softmax attention over
// positions 0..pos with kv head h/4, sigmoid output gate.
//
// Split-K flash decode.  Workgroup (b, g, split) of qm_gqa_decode_split owns
// `chunk` cache positions of kv head g and all four query heads of g, so
// each K/V byte is read from HBM once per step (the reference re-reads the
// cache once per query head, gemv.rs:963-986).  qm_gqa_decode_merge then
// merges the split partials of each (b, g) and applies the gate; with a
// single split the first kernel finishes the job itself.  The two-kernel
// form is deliberate: handing partials to a last-arriving workgroup inside
// one kernel needs agent-scope fences (an L2 writeback per workgroup), which
// measured ~1.8 us of serialized L2 time per workgroup.
//
// The kernel is an HBM stream.  Each wave walks 16-key rounds; the K and V
// rows of round r+1 are issued into a second register set before round r is
// computed (a scheduling barrier keeps the compiler from sinking them), so
// 16-32 KB per wave stay in flight.
//   QK^T: MFMA v_mfma_f32_16x16x32_f16.  q is fp32 in the reference, so it
//         enters as a two-term f16 split q ~ q_hi + q_lo (A rows 0..3 hi,
//         rows 4..7 lo).  The pair carries about 22 of fp32's 24 mantissa
//         bits (fewer when q_lo falls in the f16 subnormal range, i.e. for
//         |q| below ~2^-4); each f16 x f16 product is exact in the fp32
//         accumulator, so the score error is that split's residue, ~2^-22
//         relative.  K comes straight from the f16 cache as the B operand.
//   PV:   VALU; each lane owns 4 of the 256 dims of all four heads; the 64
//         probabilities of a round are broadcast through LDS.
#include "qm_device.h"
#include "qm_kernel_args.h"
#include "qm_gqa_common.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

#define GQA_PART_STRIDE 260   // acc[256], m, l, pad[2]

struct RoundBuf {
    half8 k[8];     // B operand: key (lane & 15), dims 64*(lane>>4) + 8*s .. +7
    uint2 v[16];    // V rows of the 16 keys, dims 4*lane .. 4*lane+3
};

// Issue the loads of one 16-key round (keys t0..t0+15, clamped to t_last so
// every address is inside the cache; clamped keys are masked later).
QM_DEV void load_round(RoundBuf& rb, const uint16_t* kbase, const uint16_t* vbase, int t0,
                       int t_last, int arow, int aq, int lane) {
    const int tk = min(t0 + arow, t_last);
    const uint16_t* krow = kbase + (size_t)tk * QM_GQA_HD + 64 * aq;
#pragma unroll
    for (int s = 0; s < 8; ++s) rb.k[s] = *reinterpret_cast<const half8*>(krow + 8 * s);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int tv = min(t0 + j, t_last);
        rb.v[j] = *reinterpret_cast<const uint2*>(vbase + (size_t)tv * QM_GQA_HD + 4 * lane);
    }
}

struct WaveState {
    float m[4], l[4], acc[4][4];
};

// One 16-key round: scores on MFMA, online softmax, PV on VALU.  The
// softmax runs in base 2: scores are scaled by log2(e)/16 and exponentiated
// with v_exp_f32 (2^x, 1 ulp), so the running max m and the partials'
// maxima are in log2 units; libm's expf per head and round was most of a
// batch-1 step's VALU time (each wave64 VALU op takes 4 cycles on a
// 16-lane SIMD, and at batch 1 one wave per SIMD does the whole round).
QM_DEV void compute_round(WaveState& st, const RoundBuf& rb, const half8 (&afr)[8], int t0,
                          int t_end, int lane, float4* pw /* LDS [16] of this wave */) {
    floatx4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 8; ++s) c = __builtin_amdgcn_mfma_f32_16x16x32_f16(afr[s], rb.k[s], c, 0, 0, 0);
    // D[i][j] sits in lane j + 16*(i/4), element i%4: lanes 0..15 carry the
    // hi rows, lanes 16..31 the lo rows of key j = lane & 15.
    const bool valid = (lane < 16) && (t0 + (lane & 15) < t_end);
    const float scale = 1.4426950408889634f / 16.0f;   // log2(e) / sqrt(256)
    float p[4], corr[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        const float sc = sum_xor16(c[h]) * scale;
        const float x = valid ? sc : -INFINITY;
        const float mt = readlane_f32(row_max16(x), 0);
        const float m_new = fmaxf(st.m[h], mt);
        corr[h] = (st.m[h] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(st.m[h] - m_new);
        p[h] = valid ? __builtin_amdgcn_exp2f(sc - m_new) : 0.0f;
        const float ps = readlane_f32(row_sum16(p[h]), 0);
        st.l[h] = st.l[h] * corr[h] + ps;
        st.m[h] = m_new;
    }
    if (lane < 16) pw[lane] = make_float4(p[0], p[1], p[2], p[3]);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int h = 0; h < 4; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e) st.acc[h][e] *= corr[h];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const float4 pj = pw[j];
        const float v0 = f16_to_f32((uint16_t)(rb.v[j].x & 0xffffu));
        const float v1 = f16_to_f32((uint16_t)(rb.v[j].x >> 16));
        const float v2 = f16_to_f32((uint16_t)(rb.v[j].y & 0xffffu));
        const float v3 = f16_to_f32((uint16_t)(rb.v[j].y >> 16));
        const float ph[4] = {pj.x, pj.y, pj.z, pj.w};
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            st.acc[h][0] = fmaf(ph[h], v0, st.acc[h][0]);
            st.acc[h][1] = fmaf(ph[h], v1, st.acc[h][1]);
            st.acc[h][2] = fmaf(ph[h], v2, st.acc[h][2]);
            st.acc[h][3] = fmaf(ph[h], v3, st.acc[h][3]);
        }
    }
    // pw is rewritten next round: order those writes after these reads.
    __builtin_amdgcn_wave_barrier();
}

// The output gate of query head qh, dims 4*lane .. 4*lane+3 (gemv.rs:1008-1011),
// loaded ahead of the attention so its latency is hidden.
QM_DEV float4 gqa_gate(const GqaDecodeArgs& A, int b, int qh, int lane) {
    return ld4(A.q_gate + ((size_t)b * QM_GQA_HEADS + qh) * (2 * QM_GQA_HD) + QM_GQA_HD + 4 * lane);
}

// Gate and store one head's output: out = (acc / l) * sigmoid(gate)
// (v_rcp_f32 / v_exp_f32, about 1 ulp each).
QM_DEV void gqa_store_out(const GqaDecodeArgs& A, int b, int qh, int lane, float4 o, float Ls,
                          float4 gv) {
    const float inv = __builtin_amdgcn_rcpf(Ls);
    float4 r;
    r.x = (o.x * inv) * sigmoid_fast(gv.x);
    r.y = (o.y * inv) * sigmoid_fast(gv.y);
    r.z = (o.z * inv) * sigmoid_fast(gv.z);
    r.w = (o.w * inv) * sigmoid_fast(gv.w);
    st4(A.out + ((size_t)b * QM_GQA_HEADS + qh) * QM_GQA_HD + 4 * lane, r);
}

extern "C" __global__ __launch_bounds__(256) void qm_gqa_decode_split(GqaDecodeArgs A) {
    __shared__ float qs[4][QM_GQA_HD];          // normed+roped q, heads 4g..4g+3
    __shared__ float wacc[4][4][QM_GQA_HD];     // per-wave partial PV
    __shared__ float4 pbuf[4][16];              // per-wave probabilities of a round
    __shared__ float wm[4][4], wl[4][4];

    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int bid = blockIdx.x;
    const int split = bid % A.nsplit;
    const int bg = bid / A.nsplit;
    const int g = bg % QM_GQA_KV_HEADS;
    const int b = bg / QM_GQA_KV_HEADS;
    const int t_begin = split * A.chunk;
    const size_t kv_base = ((size_t)b * QM_GQA_KV_HEADS + g) * (size_t)A.cap * QM_GQA_HD;
    const uint16_t* kbase = A.k_cache + kv_base;
    const uint16_t* vbase = A.v_cache + kv_base;

    // 4a. Wave w takes rounds t_begin + 64*r + 16*w (r = 0 .. nr-1).  The
    //     first round is issued before pos has arrived, bounded by max_pos
    //     (pos <= max_pos), so it overlaps the pos load and the q
    //     preparation; keys past the real end are masked when the round is
    //     computed.  The split that appends loads it again after the append.
    //     (Issuing the second round here as well measured 2% slower at batch 1.)
    const int arow = lane & 15, aq = lane >> 4;
    RoundBuf ra, rb;
    {
        const int t_end0 = min(t_begin + A.chunk, A.max_pos + 1);
        if (t_begin + 16 * w < t_end0) load_round(ra, kbase, vbase, t_begin + 16 * w, t_end0 - 1, arow, aq, lane);
    }
    float4 gv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (A.nsplit == 1) gv = gqa_gate(A, b, 4 * g + w, lane);

    int pos = A.pos ? A.pos[b] : A.max_pos;
    pos = pos < 0 ? 0 : (pos > A.max_pos ? A.max_pos : pos);
    const int L = pos + 1;
    const int t_end = min(t_begin + A.chunk, L);
    const float* cos_row = A.rope_cos + (size_t)pos * (QM_GQA_ROT / 2);
    const float* sin_row = A.rope_sin + (size_t)pos * (QM_GQA_ROT / 2);
    const bool appends = (t_begin <= pos && pos < t_end);
    const int span = t_end - t_begin - 16 * w;
    const int nr = __builtin_amdgcn_readfirstlane(span > 0 ? (span + 63) / 64 : 0);
    const int t_last = t_end - 1;

    // 1. q prep: wave w handles query head 4g+w (gemv.rs:927-949).  Every
    //    load of the q and k / v preparation is issued before any of their
    //    arithmetic, so the chain waits for one memory round trip.
    const float* qg = A.q_gate + ((size_t)b * QM_GQA_HEADS + 4 * g + w) * (2 * QM_GQA_HD);
    const float4 qx = ld4(qg + 4 * lane);
    const uint2 gq = *reinterpret_cast<const uint2*>(A.q_norm + 4 * lane);
    float4 rc, rs;
    rope_row_loads(cos_row, sin_row, lane, rc, rs);
    float4 ax = make_float4(0.0f, 0.0f, 0.0f, 0.0f);     // new k (wave 0) or v (wave 1)
    uint2 gk = make_uint2(0, 0);
    if (appends && w < 2) {
        const float* src = (w == 0 ? A.k_new : A.v_new) + ((size_t)b * QM_GQA_KV_HEADS + g) * QM_GQA_HD;
        ax = ld4(src + 4 * lane);
        gk = *reinterpret_cast<const uint2*>(A.k_norm + 4 * lane);
    }
    {
        float4 x = norm_rope_head(qx, gq, rc, rs, lane);
        *reinterpret_cast<float4*>(&qs[w][4 * lane]) = x;
    }
    // 2. The split that holds position pos appends the new k, v (gemv.rs:946-956).
    if (appends) {
        if (w == 0) {
            float4 x = norm_rope_head(ax, gk, rc, rs, lane);
            uint2 o;
            o.x = (uint32_t)f32_to_f16(x.x) | ((uint32_t)f32_to_f16(x.y) << 16);
            o.y = (uint32_t)f32_to_f16(x.z) | ((uint32_t)f32_to_f16(x.w) << 16);
            *reinterpret_cast<uint2*>(A.k_cache + kv_base + (size_t)pos * QM_GQA_HD + 4 * lane) = o;
        } else if (w == 1) {
            uint2 o;
            o.x = (uint32_t)f32_to_f16(ax.x) | ((uint32_t)f32_to_f16(ax.y) << 16);
            o.y = (uint32_t)f32_to_f16(ax.z) | ((uint32_t)f32_to_f16(ax.w) << 16);
            *reinterpret_cast<uint2*>(A.v_cache + kv_base + (size_t)pos * QM_GQA_HD + 4 * lane) = o;
        }
        // Make the appended row visible to the other waves' loads below.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    }
    __syncthreads();
    if (appends) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        if (nr > 0) load_round(ra, kbase, vbase, t_begin + 16 * w, t_last, arow, aq, lane);
    }

    // 3. A operand: row i (= lane & 15) is q_hi of head i (i < 4), q_lo of
    //    head i-4 (4 <= i < 8), zero otherwise.  K-step s, lane group
    //    aq = lane >> 4 and element e map to head dim 64*aq + 8*s + e; the B
    //    operand uses the same map, so lane group aq streams a contiguous
    //    128-byte quarter of each key row.
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

    WaveState st;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        st.m[h] = -INFINITY; st.l[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) st.acc[h][e] = 0.0f;
    }

    // 4b. Stream the rounds, next round's loads in flight during compute.
    float4* pw = pbuf[w];
    for (int r = 0; r < nr; r += 2) {
        const int t0 = t_begin + 64 * r + 16 * w;
        if (r + 1 < nr) load_round(rb, kbase, vbase, t0 + 64, t_last, arow, aq, lane);
        __builtin_amdgcn_sched_barrier(0);
        compute_round(st, ra, afr, t0, t_end, lane, pw);
        if (r + 1 >= nr) break;
        if (r + 2 < nr) load_round(ra, kbase, vbase, t0 + 128, t_last, arow, aq, lane);
        __builtin_amdgcn_sched_barrier(0);
        compute_round(st, rb, afr, t0 + 64, t_end, lane, pw);
    }

    // 5. Merge the four waves, write this split's partial.
    if (lane == 0) {
#pragma unroll
        for (int h = 0; h < 4; ++h) { wm[w][h] = st.m[h]; wl[w][h] = st.l[h]; }
    }
#pragma unroll
    for (int h = 0; h < 4; ++h)
        *reinterpret_cast<float4*>(&wacc[w][h][4 * lane]) =
            make_float4(st.acc[h][0], st.acc[h][1], st.acc[h][2], st.acc[h][3]);
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
            const float f = (wm[ww][h] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(wm[ww][h] - M);
            Ls += wl[ww][h] * f;
            const float4 a = *reinterpret_cast<const float4*>(&wacc[ww][h][4 * lane]);
            o.x += a.x * f; o.y += a.y * f; o.z += a.z * f; o.w += a.w * f;
        }
        if (A.nsplit == 1) {
            gqa_store_out(A, b, 4 * g + h, lane, o, Ls, gv);
        } else {
            float* P = A.partial + ((((size_t)b * QM_GQA_KV_HEADS + g) * A.nsplit + split) * 4 + h) * GQA_PART_STRIDE;
            st4(P + 4 * lane, o);
            if (lane == 0) { P[256] = M; P[257] = Ls; }
        }
    }
}

// Merge the split partials of query head 4g+h of sequence b and apply the
// gate.  Workgroup (b, g, h) has 16 waves; wave w folds splits w, w+16,
// w+32, w+48 (then the next 64, ...) with all four partials' loads in
// flight, so up to 64 splits cost one memory round trip, and the 16 wave
// results combine through LDS.  Lane l owns dims 4l .. 4l+3.
extern "C" __global__ __launch_bounds__(1024) void qm_gqa_decode_merge(GqaDecodeArgs A) {
    __shared__ float4 wo[16][64];
    __shared__ float wm[16], wl[16];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int h = blockIdx.x & 3;
    const int g = (blockIdx.x >> 2) % QM_GQA_KV_HEADS;
    const int b = blockIdx.x / (4 * QM_GQA_KV_HEADS);
    const int nsplit = A.nsplit;
    float4 gv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (w == 0) gv = gqa_gate(A, b, 4 * g + h, lane);
    const float* P0 = A.partial + (((size_t)b * QM_GQA_KV_HEADS + g) * nsplit * 4 + h) * GQA_PART_STRIDE;
    const size_t step = 4 * GQA_PART_STRIDE;

    float mw = -INFINITY, lw = 0.0f;
    float4 ow = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int s0 = w; s0 < nsplit; s0 += 64) {
        float4 a[4];
        float ms[4], ls[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int s = s0 + 16 * j;
            const bool ok = s < nsplit;                  // wave-uniform
            const float* P = P0 + (size_t)(ok ? s : s0) * step;
            a[j] = ld4(P + 4 * lane);
            ms[j] = ok ? P[256] : -INFINITY;
            ls[j] = P[257];
        }
        // empty splits (sequence shorter than max_pos) carry m = -inf
        const float nm = fmaxf(mw, fmaxf(fmaxf(ms[0], ms[1]), fmaxf(ms[2], ms[3])));
        if (nm == -INFINITY) continue;                   // wave-uniform
        const float c = __builtin_amdgcn_exp2f(mw - nm); // 0 while mw = -inf (log2 units)
        lw *= c;
        ow.x *= c; ow.y *= c; ow.z *= c; ow.w *= c;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float f = (ms[j] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(ms[j] - nm);
            lw = fmaf(ls[j], f, lw);
            ow.x = fmaf(a[j].x, f, ow.x);
            ow.y = fmaf(a[j].y, f, ow.y);
            ow.z = fmaf(a[j].z, f, ow.z);
            ow.w = fmaf(a[j].w, f, ow.w);
        }
        mw = nm;
    }
    if (lane == 0) { wm[w] = mw; wl[w] = lw; }
    wo[w][lane] = ow;
    __syncthreads();
    if (w == 0) {
        float M = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < 16; ++ww) M = fmaxf(M, wm[ww]);
        float Ls = 0.0f;
        float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int ww = 0; ww < 16; ++ww) {
            const float f = (wm[ww] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(wm[ww] - M);
            const float4 x = wo[ww][lane];
            Ls = fmaf(wl[ww], f, Ls);
            o.x = fmaf(x.x, f, o.x); o.y = fmaf(x.y, f, o.y);
            o.z = fmaf(x.z, f, o.z); o.w = fmaf(x.w, f, o.w);
        }
        gqa_store_out(A, b, 4 * g + h, lane, o, Ls, gv);
    }
}
