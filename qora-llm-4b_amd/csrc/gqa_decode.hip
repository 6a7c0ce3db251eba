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
// 16-32 KB per wave stay in flight.  At batch 1 the step is latency-bound
// (about one wave per SIMD), so the per-round VALU work is what the layout
// below minimises.  Both products run on MFMA, and the
// score layout of the first is the A-operand layout of the second, so the
// probabilities never leave their lanes:
//   QK^T: S = K Q^T on v_mfma_f32_16x16x32_f16 (A = 16 keys from the f16
//         cache, B = the query columns).  q is fp32 in the reference, so it
//         enters as a two-term f16 split q ~ q_hi + q_lo (columns 0..3 hi,
//         8..11 lo, the rest zero).  The pair carries about 22 of fp32's 24
//         mantissa bits (fewer when q_lo falls in the f16 subnormal range,
//         i.e. for |q| below ~2^-4); each f16 x f16 product is exact in the
//         fp32 accumulator, so the score error is that split's residue,
//         ~2^-22 relative.  Lane l ends with keys 4(l>>4)..+3 of column
//         l&15, and one row_ror:8 DPP add joins the hi and lo columns.
//   softmax: base 2 (scores scaled by log2(e)/16, v_exp_f32), all four heads
//         at once: a head's 16 scores sit in 4 lanes x 4 elements, so its max
//         and sum are 3 in-lane ops and two lane swaps (l^16, l^32).
//   PV:   O = P V on v_mfma_f32_16x16x16_f16, one instruction per 16
//         output dims (m = 0..15: B column j is dim 16j+m, so each lane
//         loads 32 contiguous bytes of a V row).  P enters as the same
//         hi/lo split (rows 0..3 hi, 8..11 lo); V is exact f16.  Keys past the
//         sequence end get p = 0 and, in a round that has any, V = 0, so cache
//         rows beyond pos never reach the sum whatever they hold.
#include "qm_device.h"
#include "qm_kernel_args.h"
#include "qm_gqa_common.h"

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

#define GQA_PART_STRIDE 260   // acc[256], m, l, pad[2]

struct RoundBuf {
    half8 k[8];      // QK A operand: key (lane & 15), dims 64*(lane>>4) + 8*s .. +7
    uint4 v[4][2];   // V rows of keys 4*(lane>>4) + i, dims 16*(lane&15) .. +15 (f16 pairs)
};

// Issue the loads of one 16-key round (keys t0..t0+15, clamped to t_last so
// every address is inside the cache; clamped keys are masked later).
QM_DEV void load_round(RoundBuf& rb, const uint16_t* kbase, const uint16_t* vbase, int t0,
                       int t_last, int lane) {
    const int c = lane & 15, grp = lane >> 4;
    const int tk = min(t0 + c, t_last);
    const uint16_t* krow = kbase + (size_t)tk * QM_GQA_HD + 64 * grp;
#pragma unroll
    for (int s = 0; s < 8; ++s) rb.k[s] = *reinterpret_cast<const half8*>(krow + 8 * s);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int tv = min(t0 + 4 * grp + i, t_last);
        const uint16_t* vrow = vbase + (size_t)tv * QM_GQA_HD + 16 * c;
        rb.v[i][0] = *reinterpret_cast<const uint4*>(vrow);
        rb.v[i][1] = *reinterpret_cast<const uint4*>(vrow + 8);
    }
}

// Per-lane online-softmax state of column lane & 15 (head (lane & 15) & 7 for
// columns 0..3 and 8..11), and the PV accumulators: o[m] lane l element e is
// row 4(l>>4)+e (hi head e in lanes 0..15, lo head e in lanes 32..47) of
// output dims 16(l&15) + m.
struct WaveState {
    float m, l;
    floatx4 o[16];
};

// One 16-key round (keys t0..t0+15 of this wave, valid below t_end).
// qsrc: this lane's B-operand column of the q block in LDS (re-read each
// round rather than held: 32 registers fewer keeps two waves per SIMD).
// The split that appends holds the new k, v rows in LDS (knew / vnew, the f16
// bits it stores to the cache); the round that contains position ap takes
// them from there instead of from the loads, which may have been issued
// before the store (so no fence or reload is needed).
QM_DEV uint32_t dword_of(const uint4 (&v)[2], int m) {   // the f16 pair holding dim m (m = 0..15)
    const uint4& u = v[m >> 3];
    const int j = (m >> 1) & 3;
    return j == 0 ? u.x : (j == 1 ? u.y : (j == 2 ? u.z : u.w));
}
QM_DEV void compute_round(WaveState& st, RoundBuf& rb, const uint16_t* qsrc, int t0, int t_end,
                          int lane, bool first, int ap, const uint16_t* knew, const uint16_t* vnew) {
    const int c = lane & 15, grp = lane >> 4;
    const int jp = ap - t0;
    if (jp >= 0 && jp < 16) {                      // uniform: the appended row is in this round
        if (c == jp) {
#pragma unroll
            for (int s = 0; s < 8; ++s) rb.k[s] = *reinterpret_cast<const half8*>(knew + 64 * grp + 8 * s);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (4 * grp + i == jp) {
                rb.v[i][0] = *reinterpret_cast<const uint4*>(vnew + 16 * c);
                rb.v[i][1] = *reinterpret_cast<const uint4*>(vnew + 16 * c + 8);
            }
        }
    }
    floatx4 sacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 8; ++s)
        sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(rb.k[s], *reinterpret_cast<const half8*>(qsrc + 8 * s),
                                                      sacc, 0, 0, 0);
    const float scale = 1.4426950408889634f / 16.0f;   // log2(e) / sqrt(256)
    const int kbase = t0 + 4 * grp;
    float x[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float sc = (sacc[e] + dpp_f32<0x128>(sacc[e])) * scale;   // hi + lo column
        x[e] = (kbase + e < t_end) ? sc : -INFINITY;
    }
    float mx = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    mx = max_xor32(max_xor16(mx));
    const float m_new = fmaxf(st.m, mx);
    // A fully masked round leaves m_new = -inf for a fresh state: p = 0 then.
    const float corr = (st.m == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(st.m - m_new);
    float p[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) p[e] = (x[e] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(x[e] - m_new);
    const float ps = sum_xor32(sum_xor16((p[0] + p[1]) + (p[2] + p[3])));
    st.l = st.l * corr + ps;
    st.m = m_new;

    // Rescale the accumulators: o row e carries head e, whose factor sits in
    // lane e.  Skipped (uniformly) while every head's maximum is unchanged.
    //  The first round's accumulators are still zero.
    const float c0 = readlane_f32(corr, 0), c1 = readlane_f32(corr, 1);
    const float c2 = readlane_f32(corr, 2), c3 = readlane_f32(corr, 3);
    if (!first && (c0 != 1.0f || c1 != 1.0f || c2 != 1.0f || c3 != 1.0f)) {
#pragma unroll
        for (int m = 0; m < 16; ++m) {
            st.o[m][0] *= c0; st.o[m][1] *= c1; st.o[m][2] *= c2; st.o[m][3] *= c3;
        }
    }

    // P operand: row c = hi (c < 4) or lo (8 <= c < 12) part of head c & 7's
    // probabilities of keys 4*grp .. +3, zero in the other rows.
    half4 pa;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const _Float16 hi = (_Float16)p[e];
        const _Float16 lo = (_Float16)(p[e] - (float)hi);
        pa[e] = c < 4 ? hi : ((c >= 8 && c < 12) ? lo : (_Float16)0.0f);
    }
    // Keys at or past t_end: zero their V rows (uniform test; tail rounds only).
    if (t0 + 16 > t_end) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (kbase + i >= t_end) { rb.v[i][0] = make_uint4(0, 0, 0, 0); rb.v[i][1] = make_uint4(0, 0, 0, 0); }
        }
    }
    // B operand of output dim 16c + m: the f16 at dim m of the four key rows,
    // packed pairwise with v_perm_b32 (low halves for even m, high for odd).
#pragma unroll
    for (int m = 0; m < 16; ++m) {
        const uint32_t sel = (m & 1) ? 0x07060302u : 0x05040100u;
        uint2 vb;
        vb.x = __builtin_amdgcn_perm(dword_of(rb.v[1], m), dword_of(rb.v[0], m), sel);
        vb.y = __builtin_amdgcn_perm(dword_of(rb.v[3], m), dword_of(rb.v[2], m), sel);
        st.o[m] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(half4, vb), st.o[m], 0, 0, 0);
    }
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

QM_DEV uint2 pack_f16x4(float a, float b, float c, float d) {
    uint2 o;
    o.x = (uint32_t)f32_to_f16(a) | ((uint32_t)f32_to_f16(b) << 16);
    o.y = (uint32_t)f32_to_f16(c) | ((uint32_t)f32_to_f16(d) << 16);
    return o;
}

template <int NW>
struct SplitLds {
    // q columns in f16: rows 0..3 q_hi of heads 4g..4g+3, rows 4..7 q_lo,
    // row 8 zeros (the B operand's unused columns).
    __attribute__((aligned(16))) uint16_t qhl[9][QM_GQA_HD];
    float wacc[NW][4][QM_GQA_HD];               // per-wave partial PV
    float wm[NW][4], wl[NW][4];
    __attribute__((aligned(16))) uint16_t knew[QM_GQA_HD], vnew[QM_GQA_HD];   // appended rows
};

// POS_ARG: no per-sequence positions (every sequence at max_pos, as at batch
// 1), so the RoPE rows and the append's inputs are known before any load and
// are issued with the q row, ahead of the first round; otherwise they wait
// for pos and follow the round.
// NW: waves per workgroup (4 to 8).  Waves 0..3 also own the q prep and the
// final merge of query heads 4g..4g+3; every wave streams rounds.  Short
// splits (chunk = 16 NW keys, as at batch 1) thus take one round per wave.
template <bool POS_ARG, int NW>
QM_DEV void split_body(const GqaDecodeArgs& A, SplitLds<NW>& sh) {
    auto& qhl = sh.qhl;
    auto& wacc = sh.wacc;
    auto& wm = sh.wm;
    auto& wl = sh.wl;
    auto& knew = sh.knew;
    auto& vnew = sh.vnew;
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

    // Loads first, in the order their consumers need them: pos (scalar), the
    // q row and its norm weight (and, with POS_ARG, the RoPE rows and the
    // appended k / v), then the first 16-key round (bounded by max_pos,
    // since pos <= max_pos; keys past the real end are masked when the round
    // is computed), then what depends on a loaded pos.  Each wave's vector
    // loads complete in issue order, so the q norm starts while the round is
    // still in flight.
    int pos = POS_ARG ? A.max_pos : A.pos[b];
    const float* qg = A.q_gate + ((size_t)b * QM_GQA_HEADS + 4 * g + (w & 3)) * (2 * QM_GQA_HD);
    const float4 qx = ld4(qg + 4 * lane);
    const uint2 gq = *reinterpret_cast<const uint2*>(A.q_norm + 4 * lane);
    float4 rc, rs;
    float4 ax = make_float4(0.0f, 0.0f, 0.0f, 0.0f);     // new k (wave 0) or v (wave 1)
    uint2 gk = make_uint2(0, 0);
    auto pos_loads = [&](int p, bool app) {
        rope_row_loads(A.rope_cos + (size_t)p * (QM_GQA_ROT / 2), A.rope_sin + (size_t)p * (QM_GQA_ROT / 2), lane, rc, rs);
        if (app && w < 2) {
            const float* src = (w == 0 ? A.k_new : A.v_new) + ((size_t)b * QM_GQA_KV_HEADS + g) * QM_GQA_HD;
            ax = ld4(src + 4 * lane);
            gk = *reinterpret_cast<const uint2*>(A.k_norm + 4 * lane);
        }
    };
    if (POS_ARG) {
        const int t_end = min(t_begin + A.chunk, pos + 1);
        pos_loads(pos, t_begin <= pos && pos < t_end);
    }
    __builtin_amdgcn_sched_barrier(0);
    // 4a. Wave w takes rounds t_begin + 16*NW*r + 16*w (r = 0 .. nr-1).
    RoundBuf ra, rb;
    {
        const int t_end0 = min(t_begin + A.chunk, A.max_pos + 1);
        if (t_begin + 16 * w < t_end0) load_round(ra, kbase, vbase, t_begin + 16 * w, t_end0 - 1, lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    pos = pos < 0 ? 0 : (pos > A.max_pos ? A.max_pos : pos);
    const int L = pos + 1;
    const int t_end = min(t_begin + A.chunk, L);
    const bool appends = (t_begin <= pos && pos < t_end);
    const int span = t_end - t_begin - 16 * w;
    const int nr = __builtin_amdgcn_readfirstlane(span > 0 ? (span + 16 * NW - 1) / (16 * NW) : 0);
    const int t_last = t_end - 1;
    if (!POS_ARG) pos_loads(pos, appends);
    float4 gv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (A.nsplit == 1) gv = gqa_gate(A, b, 4 * g + (w & 3), lane);

    // 1. q prep: wave w < 4 handles query head 4g+w (gemv.rs:927-949),
    //    stored as its f16 hi / lo parts.
    if (w < 4) {
        const float4 x = norm_rope_head(qx, gq, rc, rs, lane);
        const uint2 hi = pack_f16x4(x.x, x.y, x.z, x.w);
        const float4 xh = make_float4(f16_to_f32((uint16_t)(hi.x & 0xffffu)), f16_to_f32((uint16_t)(hi.x >> 16)),
                                      f16_to_f32((uint16_t)(hi.y & 0xffffu)), f16_to_f32((uint16_t)(hi.y >> 16)));
        *reinterpret_cast<uint2*>(&qhl[w][4 * lane]) = hi;
        *reinterpret_cast<uint2*>(&qhl[4 + w][4 * lane]) = pack_f16x4(x.x - xh.x, x.y - xh.y, x.z - xh.z, x.w - xh.w);
        if (w == 3) *reinterpret_cast<uint2*>(&qhl[8][4 * lane]) = make_uint2(0, 0);
    }
    // 2. The split that holds position pos appends the new k, v (gemv.rs:946-956);
    //    its rounds take the rows from LDS.
    if (appends) {
        if (w == 0) {
            const float4 x = norm_rope_head(ax, gk, rc, rs, lane);
            const uint2 o = pack_f16x4(x.x, x.y, x.z, x.w);
            *reinterpret_cast<uint2*>(A.k_cache + kv_base + (size_t)pos * QM_GQA_HD + 4 * lane) = o;
            *reinterpret_cast<uint2*>(&knew[4 * lane]) = o;
        } else if (w == 1) {
            const uint2 o = pack_f16x4(ax.x, ax.y, ax.z, ax.w);
            *reinterpret_cast<uint2*>(A.v_cache + kv_base + (size_t)pos * QM_GQA_HD + 4 * lane) = o;
            *reinterpret_cast<uint2*>(&vnew[4 * lane]) = o;
        }
    }
    const int ap = __builtin_amdgcn_readfirstlane(appends ? pos : -0x40000000);
    __syncthreads();

    // 3. B operand of QK: column c = lane & 15 is q_hi of head c (c < 4),
    //    q_lo of head c-8 (8 <= c < 12), zero otherwise.  K-step s, lane
    //    group lane >> 4 and element e map to head dim 64*(lane>>4) + 8*s + e,
    //    as in the A operand (so lane group j streams a contiguous 128-byte
    //    quarter of each key row).
    const uint16_t* qsrc;
    {
        const int c = lane & 15;
        const int row = c < 4 ? c : ((c >= 8 && c < 12) ? c - 4 : 8);
        qsrc = &qhl[row][64 * (lane >> 4)];
    }

    WaveState st;
    st.m = -INFINITY;
    st.l = 0.0f;
#pragma unroll
    for (int m = 0; m < 16; ++m) st.o[m] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    // 4b. Stream the rounds, next round's loads in flight during compute.
    for (int r = 0; r < nr; r += 2) {
        const int t0 = t_begin + 16 * NW * r + 16 * w;
        if (r + 1 < nr) load_round(rb, kbase, vbase, t0 + 16 * NW, t_last, lane);
        __builtin_amdgcn_sched_barrier(0);
        compute_round(st, ra, qsrc, t0, t_end, lane, r == 0, ap, knew, vnew);
        if (r + 1 >= nr) break;
        if (r + 2 < nr) load_round(ra, kbase, vbase, t0 + 32 * NW, t_last, lane);
        __builtin_amdgcn_sched_barrier(0);
        compute_round(st, rb, qsrc, t0 + 16 * NW, t_end, lane, false, ap, knew, vnew);
    }

    // 5. Join each head's hi and lo rows (lanes l and l^32: one row swap per
    //    pair of accumulators), merge the four waves, write this split's
    //    partial.  After the swap-add of (o[m][e], o[m][e+1]), lanes 0..15
    //    hold head e and lanes 32..47 head e+1 of dims 16(l&15) + m.
    if (lane < 4) { wm[w][lane] = st.m; wl[w][lane] = st.l; }
    {
        const int c = lane & 15;
        const bool writer = (lane & 16) == 0;
        const int hsel = lane >> 5;                  // 0: lanes 0..31, 1: lanes 32..63
#pragma unroll
        for (int ep = 0; ep < 4; ep += 2) {
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                float r4[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int m = 4 * q4 + k;
                    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(st.o[m][ep]),
                                                                     __float_as_uint(st.o[m][ep + 1]), false, false);
                    r4[k] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
                }
                if (writer)
                    *reinterpret_cast<float4*>(&wacc[w][ep + hsel][16 * c + 4 * q4]) =
                        make_float4(r4[0], r4[1], r4[2], r4[3]);
            }
        }
    }
    __syncthreads();
    if (w < 4) {
        const int h = w;                      // thread (h, lane): dims 4*lane..+3
        float M = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, wm[ww][h]);
        float Ls = 0.0f;
        float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int ww = 0; ww < NW; ++ww) {
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

template <int NW>
QM_DEV void split_kernel(const GqaDecodeArgs& A) {
    __shared__ SplitLds<NW> sh;
    if (A.pos) split_body<false, NW>(A, sh);
    else split_body<true, NW>(A, sh);
}
extern "C" __global__ __launch_bounds__(256) void qm_gqa_decode_split(GqaDecodeArgs A) { split_kernel<4>(A); }
extern "C" __global__ __launch_bounds__(320) void qm_gqa_decode_split_w5(GqaDecodeArgs A) { split_kernel<5>(A); }
extern "C" __global__ __launch_bounds__(384) void qm_gqa_decode_split_w6(GqaDecodeArgs A) { split_kernel<6>(A); }
extern "C" __global__ __launch_bounds__(448) void qm_gqa_decode_split_w7(GqaDecodeArgs A) { split_kernel<7>(A); }
extern "C" __global__ __launch_bounds__(512) void qm_gqa_decode_split_w8(GqaDecodeArgs A) { split_kernel<8>(A); }

// Merge the split partials of query head 4g+h of sequence b and apply the
// gate.  One wave per (b, g, h, quarter of the dims): lane l owns dim
// 64 q + l.  The splits are folded 56 at a time with every load of a batch in
// flight at once (a wave can have 63 vector loads outstanding): each lane
// loads its dim of the batch's partials and one split's (max, sum) pair; the
// batch maximum and the sum of the rescaled sums are wave reductions, and
// split j's factor is read from lane j.  So up to 56 splits cost one memory
// round trip, and the merge needs no LDS or barrier.  (Two waves splitting
// the splits, with an LDS combine, measured no faster at batch 1.)
#define MERGE_BATCH 56
QM_DEV float wave_max64(float x) {
    return max_xor32(max_xor16(row_max16(x)));
}
extern "C" __global__ __launch_bounds__(64) void qm_gqa_decode_merge(GqaDecodeArgs A) {
    const int lane = threadIdx.x;
    const int q = blockIdx.x & 3;
    const int h = (blockIdx.x >> 2) & 3;
    const int g = (blockIdx.x >> 4) % QM_GQA_KV_HEADS;
    const int b = blockIdx.x / (16 * QM_GQA_KV_HEADS);
    const int nsplit = A.nsplit;
    const int d = 64 * q + lane;
    const float gate = A.q_gate[((size_t)b * QM_GQA_HEADS + 4 * g + h) * (2 * QM_GQA_HD) + QM_GQA_HD + d];
    const float* P0 = A.partial + (((size_t)b * QM_GQA_KV_HEADS + g) * nsplit * 4 + h) * GQA_PART_STRIDE;
    const size_t step = 4 * GQA_PART_STRIDE;
    float M = -INFINITY, Ls = 0.0f, o = 0.0f;
    for (int s0 = 0; s0 < nsplit; s0 += MERGE_BATCH) {        // uniform
        float a[MERGE_BATCH];
#pragma unroll
        for (int j = 0; j < MERGE_BATCH; ++j) a[j] = P0[(size_t)min(s0 + j, nsplit - 1) * step + d];
        const bool mine = lane < MERGE_BATCH && s0 + lane < nsplit;       // lane's split s0 + lane
        const float2 ml = *reinterpret_cast<const float2*>(P0 + (size_t)min(s0 + lane, nsplit - 1) * step + 256);
        // empty splits (sequence shorter than max_pos) carry m = -inf
        const float mj = mine ? ml.x : -INFINITY;
        const float mb = fmaxf(M, wave_max64(mj));
        if (mb == -INFINITY) continue;                         // uniform
        const float c = __builtin_amdgcn_exp2f(M - mb);         // 0 while M = -inf (log2 units)
        const float fj = (mj == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mj - mb);
        Ls = Ls * c + wave_sum64(mine ? ml.y * fj : 0.0f);
        float op[4] = {o * c, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < MERGE_BATCH; ++j) op[j & 3] = fmaf(a[j], readlane_f32(fj, j), op[j & 3]);
        o = (op[0] + op[1]) + (op[2] + op[3]);
        M = mb;
    }
    // gemv.rs:1008-1011: out = (o / l) * sigmoid(gate)
    A.out[((size_t)b * QM_GQA_HEADS + 4 * g + h) * QM_GQA_HD + d] = (o * __builtin_amdgcn_rcpf(Ls)) * sigmoid_fast(gate);
}
