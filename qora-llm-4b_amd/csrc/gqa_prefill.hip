// gqa_prefill.hip -- full-attention GQA causal prefill for gfx950.
//
// Replaces the mixer slice of prefill_attn_layer (gemv.rs:1364-1444): per
// token QK RMSNorm (1+gamma) and partial RoPE at positions 0..S-1, the KV
// cache replaced by the normed/roped K and V (f16), causal softmax attention
// with kv head h/4, sigmoid output gate.
//
// qm_gqa_prefill_kv    K norm + RoPE -> f16 K cache; V -> f16 V cache; and
//                      both again as 64-key tiles in the attention's MFMA
//                      fragment order (K, and V transposed), so each tile
//                      is one contiguous 64 KB block.
// qm_gqa_prefill_attn  flash attention on MFMA.  A workgroup owns 48 query
//                      tokens of all four query heads of one kv group (12
//                      waves: head 4g + (w & 3), 16 rows each, three waves
//                      per SIMD), so every K / V tile staged in LDS feeds
//                      four heads.  Scores are computed transposed,
//                      S^T = K Q^T (keys x rows), with v_mfma_f32_16x16x32:
//                      a lane of an S^T fragment then holds four consecutive
//                      keys of one row, which is exactly what the PV product
//                      (rows x dims, contracting keys) needs as its A operand
//                      once two 16-key fragments are paired; the V^T operand
//                      uses the same key set per lane (the S^T rows are
//                      permuted so that set is 8 consecutive keys).  No lane
//                      shuffles between the two products.  Online softmax in
//                      base 2, fp32, with a lazily moved reference max.  K / V
//                      tiles are double-buffered in LDS and copied there, 1 KB
//                      per instruction, by LDS DMA one tile ahead of use.
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

// Key held by row i of S^T fragment kk: the four fragments of a 64-key tile
// are arranged so that, for PV k-step ks = kk >> 1, a lane's pair of
// fragments 2ks, 2ks+1 holds the 8 consecutive keys 32 ks + 8 lq .. + 7.
QM_DEV int frag_key(int kk, int i) { return 32 * (kk >> 1) + 8 * (i >> 2) + 4 * (kk & 1) + (i & 3); }

// ---------------------------------------------------------------------------
// K / V cache write (gemv.rs:1387-1400).  Workgroup = 64 tokens (one tile) of
// kv head g.  The tile copy kvf + (g * ntile + tile) * 64 KB is 64 blocks of
// 1 KB, block entry l = the 16 bytes MFMA lane l = (lr, lq) = (l & 15, l >> 4)
// reads:
//   block b < 32, b = 8 kk + s:       K row frag_key(kk, lr), dims 32 s + 8 lq .. + 7
//   block b >= 32, b - 32 = 2 dt + ks: V dim 16 dt + lr, keys 32 ks + 8 lq .. + 7
// Keys past S are zero.
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(512) void qm_gqa_prefill_kv(GqaPrefillArgs A) {
    __shared__ _Float16 ks[64][264];
    __shared__ _Float16 vs[64][264];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int g = blockIdx.x % QM_GQA_KV_HEADS;
    const int t0 = (blockIdx.x / QM_GQA_KV_HEADS) * 64;
    // the attention kernel that follows takes its row blocks from these
    if (blockIdx.x == 0 && tid < QM_GQA_KV_HEADS) A.queue[tid] = 0;
    // K: wave w (of 8) normalises and rotates tokens t0+8w .. t0+8w+7.  All
    // 8 rows are loaded (at clamped, valid rows) before any arithmetic, so
    // the wave waits for one memory round trip, not one per token.
    // V's rows are requested right after K's (their conversion waits until
    // K is done, and a wave's loads return in issue order).
    const int vi = tid >> 3, vp = tid & 7, vt = t0 + vi;
    uint4 vraw[4];
    {
        uint2 raw[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int t = min(t0 + 8 * w + j, A.S - 1);
            raw[j] = *reinterpret_cast<const uint2*>(A.k + ((size_t)t * QM_GQA_KV_HEADS + g) * QM_GQA_HD + 4 * lane);
        }
        const uint2 gw = *reinterpret_cast<const uint2*>(A.k_norm + 4 * lane);
        // RoPE rows four tokens at a time, loaded by every lane (lanes 0..15
        // use them) so no per-token branch serializes the loads; each group's
        // rows are requested one group ahead
        const int i0 = (lane & 7) * 4;
        float4 cr[2][4], sr[2][4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int tc = min(t0 + 8 * w + jj, A.S - 1);
            cr[0][jj] = ld4(A.rope_cos + (size_t)tc * 32 + i0);
            sr[0][jj] = ld4(A.rope_sin + (size_t)tc * 32 + i0);
        }
        {
            const uint16_t* vrow = A.v + ((size_t)min(vt, A.S - 1) * QM_GQA_KV_HEADS + g) * QM_GQA_HD + 8 * vp;
#pragma unroll
            for (int q = 0; q < 4; ++q) vraw[q] = *reinterpret_cast<const uint4*>(vrow + 64 * q);
        }
        const float g1[4] = {1.0f + f16_to_f32((uint16_t)(gw.x & 0xffffu)), 1.0f + f16_to_f32((uint16_t)(gw.x >> 16)),
                             1.0f + f16_to_f32((uint16_t)(gw.y & 0xffffu)), 1.0f + f16_to_f32((uint16_t)(gw.y >> 16))};
#pragma unroll
        for (int jb = 0; jb < 8; jb += 4) {
            const int cb = (jb >> 2) & 1;
            if (jb + 4 < 8) {
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const int tc = min(t0 + 8 * w + jb + 4 + jj, A.S - 1);
                    cr[cb ^ 1][jj] = ld4(A.rope_cos + (size_t)tc * 32 + i0);
                    sr[cb ^ 1][jj] = ld4(A.rope_sin + (size_t)tc * 32 + i0);
                }
            }
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const int t = t0 + 8 * w + jb + jj;
                // gemv.rs:586-597 (RMSNorm, 1 + gamma) and :604-627 (split-half RoPE)
                float4 x = bf16x4_to_f32(raw[jb + jj]);
                float ss = x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
                ss = wave_sum64(ss);
                const float inv = 1.0f / sqrtf(ss / (float)QM_GQA_HD + 1e-6f);
                x.x = x.x * inv * g1[0]; x.y = x.y * inv * g1[1];
                x.z = x.z * inv * g1[2]; x.w = x.w * inv * g1[3];
                float4 pr;                                        // rotation partner (lane ^ 8)
                pr.x = dpp_f32<0x128>(x.x); pr.y = dpp_f32<0x128>(x.y);
                pr.z = dpp_f32<0x128>(x.z); pr.w = dpp_f32<0x128>(x.w);
                // x1 c - x2 s (lanes 0..7), x2 c + x1 s (lanes 8..15)
                const float4 ps = lane < 8 ? make_float4(-pr.x, -pr.y, -pr.z, -pr.w) : pr;
                float4 y;
                y.x = x.x * cr[cb][jj].x + ps.x * sr[cb][jj].x; y.y = x.y * cr[cb][jj].y + ps.y * sr[cb][jj].y;
                y.z = x.z * cr[cb][jj].z + ps.z * sr[cb][jj].z; y.w = x.w * cr[cb][jj].w + ps.w * sr[cb][jj].w;
                if (lane < 16) x = y;
                uint2 h = make_uint2(0, 0);
                if (t < A.S) {                                    // wave-uniform
                    h = f32x4_to_f16(x);
                    *reinterpret_cast<uint2*>(A.k_cache + ((size_t)g * A.cap + t) * QM_GQA_HD + 4 * lane) = h;
                }
                *reinterpret_cast<uint2*>(&ks[8 * w + jb + jj][4 * lane]) = h;
            }
        }
    }
    // V: rows to the cache, and into LDS for the V^T tile copy.  The eight
    // threads of a token cover 64 consecutive dims per step (128-byte
    // pieces); all four raw loads (at a clamped, valid row) were issued
    // with K's.
    {
        const int i = vi, p = vp, t = vt;
        const uint4 (&raw)[4] = vraw;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint4 h16 = make_uint4(0, 0, 0, 0);
            if (t < A.S) {
                const float4 lo = bf16x4_to_f32(make_uint2(raw[q].x, raw[q].y));
                const float4 hi = bf16x4_to_f32(make_uint2(raw[q].z, raw[q].w));
                const uint2 a = f32x4_to_f16(lo), b = f32x4_to_f16(hi);
                h16 = make_uint4(a.x, a.y, b.x, b.y);
                *reinterpret_cast<uint4*>(A.v_cache + ((size_t)g * A.cap + t) * QM_GQA_HD + 64 * q + 8 * p) = h16;
            }
            *reinterpret_cast<uint4*>(&vs[i][64 * q + 8 * p]) = h16;
        }
    }
    __syncthreads();
    // the tile copy: entry p = tid + 512 i of 4096, consecutive threads on
    // consecutive 16-byte entries
    {
        uint16_t* dst = A.kvf + ((size_t)g * (A.s_pad / 64) + (t0 >> 6)) * (64 * 512);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int p = tid + 512 * i, b = p >> 6, l = p & 63, lr = l & 15, lq = l >> 4;
            const int kk = b >> 3, s8 = b & 7;
            *reinterpret_cast<half8*>(dst + 8 * p) =
                *reinterpret_cast<const half8*>(&ks[frag_key(kk, lr)][32 * s8 + 8 * lq]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int p = tid + 512 * i, b = p >> 6, l = p & 63, lr = l & 15, lq = l >> 4;
            const int d = 16 * (b >> 1) + lr, k8 = 32 * (b & 1) + 8 * lq;
            half8 hv;
#pragma unroll
            for (int e = 0; e < 8; ++e) hv[e] = vs[k8 + e][d];
            *reinterpret_cast<half8*>(dst + 32 * 512 + 8 * p) = hv;
        }
    }
}

// ---------------------------------------------------------------------------
// Flash attention.  Lane (lr, lq) = (lane & 15, lane >> 4).
// ---------------------------------------------------------------------------
// LDS (bytes): tile buffers 0, 1 of 64 KB, each the 64 KB tile copy written
// by qm_gqa_prefill_kv: K blocks (kk, s) then V^T blocks (dt, ks), block
// entry l the 16 bytes lane l reads for that product, so every fragment read
// is lane * 16 + an immediate (no bank conflicts, no per-read address
// registers).
#define SM_K(b) ((b) * 65536)
#define SM_V(b) ((b) * 65536 + 32768)
#define SM_BYTES 131072

// A row block is 48 query rows of the four query heads of one kv group: 12
// waves, wave w on head 4g + (w & 3) and rows 16 (w >> 2) .. +15, three
// waves per SIMD, so one wave's LDS and softmax latency hides behind the
// other waves' MFMAs.  Each iteration fetches the next K / V^T tile by LDS
// DMA (the tile's 64 blocks dealt round-robin over the waves), then computes
// the current tile's scores, softmax and P V.
// The kernel is persistent: one workgroup per CU, workgroup b serving kv
// group b & 3 (workgroups are dealt to the XCDs round-robin, so each XCD's L2
// holds one group's K / V).  Row blocks are drawn from a per-group atomic
// counter, so the causal triangle's unequal blocks balance across CUs (a
// fixed assignment left some CUs with a third more tiles than others).  The
// n-th draw takes block order[n] when the host passes an order (a packing of
// the blocks into the workgroups, listed by planned start time), else the
// n-th longest block.  A workgroup whose own queue is empty takes the
// remaining (short) blocks of the other groups, which evens out the XCDs'
// speeds.
#define TQ3 48

// Fragment reads in flight per wave in the two products: with 32 reads of
// 1 KB per product and three waves per SIMD, keeping 6 in flight (24 VGPRs)
// hides the LDS latency; the compiler's own order kept one or two.
#define LOOKAHEAD 6

// Orders the preceding product's 32 LDS fragment reads and its 32 + EXTRA
// MFMAs as: LOOKAHEAD reads, then (MFMA, read) pairs, then the remaining
// MFMAs.  Only an ordering hint: the waits stay the compiler's.
template <int EXTRA>
QM_DEV void sched_reads_ahead() {
    __builtin_amdgcn_sched_group_barrier(0x100, LOOKAHEAD, 0);      // DS reads
#pragma unroll
    for (int i = 0; i < 32 - LOOKAHEAD; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);          // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, LOOKAHEAD + EXTRA, 0);
}

extern "C" __global__ __launch_bounds__(768) void qm_gqa_prefill_attn(GqaPrefillAttnArgs P) {
    const GqaPrefillArgs& A = P.a;
    __shared__ __attribute__((aligned(1024))) char sm[SM_BYTES];
    __shared__ int item_s;
    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nblk = (A.S + TQ3 - 1) / TQ3;
    const uint32_t sm_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)sm;
    // item = group * nblk + block index; own group first, then the others
    // (the own group's index may already have been drawn: first)
    auto claim = [&](int g0, int first) {
        if (first < nblk) return g0 * nblk + first;
        for (int k = 1; k < QM_GQA_KV_HEADS; ++k) {
            const int gg = (g0 + k) & (QM_GQA_KV_HEADS - 1);
            const int i = atomicAdd(A.queue + gg, 1);
            if (i < nblk) return gg * nblk + i;
        }
        return -1;
    };

    const int home = blockIdx.x & (QM_GQA_KV_HEADS - 1);
    if (tid == 0) item_s = claim(home, atomicAdd(A.queue + home, 1));
    __syncthreads();
    int item = item_s;
    while (item >= 0) {                     // workgroup-uniform
        const int g = item / nblk;
        const uint16_t* tiles = A.kvf + (size_t)g * (A.s_pad / 64) * (64 * 512);
        // the next block is claimed three tiles before this one ends: late
        // enough to keep the queue's order, early enough to hide the atomic's
        // latency
        int nxt = 0;
        // lane-derived addresses are recomputed per row block (cheap)
        // rather than held across blocks, which would spill them
        int lane = tid & 63;
        asm volatile("" : "+v"(lane));
        const int lr = lane & 15, lq = lane >> 4;
        const int draw = item - g * nblk;
        const int tb = P.ordered ? (int)P.order[draw] : nblk - 1 - draw;
        const int t0 = tb * TQ3;
        const int qh = 4 * g + (w & 3);
        const int r0 = t0 + 16 * (w >> 2);
        // tiles up to the block's last row, within the zero-padded V^T copy
        const int nkt = min((t0 + TQ3 + KT - 1) / KT, A.s_pad / KT);

        // tile fetch, K half (blocks 0..31) or V^T half (32..63): block
        // h + w + 12 j, one contiguous 1 KB piece each
        auto fetch = [&](int kt, int buf, int h) {
            const uint16_t* src = tiles + (size_t)kt * (64 * 512) + 8 * lane;
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                const int b = h + w + 12 * j;
                if (b < h + 32) dma16(src + 512 * b, sm_lds + SM_K(buf) + 1024 * b);
            }
        };
        fetch(0, 0, 0);                          // in flight during the q prep
        fetch(0, 0, 32);

        // 1. q: RMSNorm (1+gamma, eps 1e-6; gemv.rs:586-597) and split-half RoPE
        //    (gemv.rs:604-627) straight into the B fragments: lane (lr, lq) holds
        //    dims 32 s + 8 lq + e of row r0 + lr, so the row's sum of squares is
        //    a reduction over the four lanes lr + 16 lq, and each rotation pair
        //    (i, i + 32), i = 8 lq + e, sits in one lane (s = 0 and s = 1).
        half8 qf[8];                            // B[k = dim][n = row]: 8 dims of row n
        {
            const int t = r0 + lr;
            const int tc = min(t, A.S - 1);     // rows past S: any valid row, then zeroed
            const uint16_t* qrow = A.q_gate + ((size_t)tc * QM_GQA_HEADS + qh) * (2 * QM_GQA_HD) + 8 * lq;
            // every load of the prep (q row, gamma, RoPE row) is issued before
            // any arithmetic, so the prep waits for one memory round trip
            uint4 u[8], gq[8];                  // the row's 64 dims of this lane, packed bf16; gamma
#pragma unroll
            for (int s = 0; s < 8; ++s) u[s] = *reinterpret_cast<const uint4*>(qrow + 32 * s);
#pragma unroll
            for (int s = 0; s < 8; ++s) gq[s] = *reinterpret_cast<const uint4*>(A.q_norm + 32 * s + 8 * lq);
            const float* crow = A.rope_cos + (size_t)tc * 32 + 8 * lq;
            const float* srow = A.rope_sin + (size_t)tc * 32 + 8 * lq;
            const float4 c0 = ld4(crow), c1 = ld4(crow + 4), s0 = ld4(srow), s1 = ld4(srow + 4);
            if (t >= A.S) {
#pragma unroll
                for (int s = 0; s < 8; ++s) u[s] = make_uint4(0, 0, 0, 0);
            }
            auto unpack = [](uint4 v, float (&x)[8]) {
                const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    x[2 * e] = bf16_to_f32((uint16_t)(wv[e] & 0xffffu));
                    x[2 * e + 1] = bf16_to_f32((uint16_t)(wv[e] >> 16));
                }
            };
            float ss = 0.0f;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                float x[8];
                unpack(u[s], x);
#pragma unroll
                for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
            }
            ss = sum_xor32(sum_xor16(ss));
            const float inv = 1.0f / sqrtf(ss / (float)QM_GQA_HD + 1e-6f);
            // the softmax scale 1/sqrt(256) in base 2 is folded into q, so the
            // scores come out of the MFMA in log2 units
            const float sl2 = (1.0f / 16.0f) * 1.4426950408889634f;
            auto normed = [&](int s, float (&x)[8]) {     // x * inv * (1 + gamma)
                unpack(u[s], x);
                const uint32_t gv[4] = {gq[s].x, gq[s].y, gq[s].z, gq[s].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    x[2 * e] = x[2 * e] * inv * (1.0f + f16_to_f32((uint16_t)(gv[e] & 0xffffu)));
                    x[2 * e + 1] = x[2 * e + 1] * inv * (1.0f + f16_to_f32((uint16_t)(gv[e] >> 16)));
                }
            };
            {
                float x1[8], x2[8];
                normed(0, x1);
                normed(1, x2);
                const float cs[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
                const float sn[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    qf[0][e] = (_Float16)((x1[e] * cs[e] - x2[e] * sn[e]) * sl2);
                    qf[1][e] = (_Float16)((x2[e] * cs[e] + x1[e] * sn[e]) * sl2);
                }
            }
#pragma unroll
            for (int s = 2; s < 8; ++s) {
                float x[8];
                normed(s, x);
#pragma unroll
                for (int e = 0; e < 8; ++e) qf[s][e] = (_Float16)(x[e] * sl2);
            }
        }

        // O[0..15]: P V; O[16]: P times a ones B operand, i.e. the row sums of
        // P (every column), in the same lane layout and rescaled with the rest
        floatx4 O[17];
#pragma unroll
        for (int dt = 0; dt < 17; ++dt) O[dt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        float m_run = -INFINITY;
        const int tok = r0 + lr;
        half8 ones;
#pragma unroll
        for (int e = 0; e < 8; ++e) ones[e] = (_Float16)1.0f;

        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // tile 0 landed (this wave's part)
        __syncthreads();                        // ... for every wave

        const int kt_claim = max(nkt - 3, 0);
        for (int kt = 0; kt < nkt; ++kt) {
            // the home queue's next index is drawn here; its latency hides
            // behind the remaining tiles, and it is resolved at the end
            if (tid == 0 && kt == kt_claim) nxt = atomicAdd(A.queue + home, 1);
            const int k0 = kt * KT, b = kt & 1;
            // the other buffer was last read before the previous barrier; the
            // V^T half is requested after the scores
            if (kt + 1 < nkt) fetch(kt + 1, b ^ 1, 0);
            const char* Kb = sm + SM_K(b);
            const char* Vb = sm + SM_V(b);

            // S^T = K Q^T: fragment kk row i is key frag_key(kk, i) of the tile.
            // k-step major, so consecutive MFMAs feed four independent
            // accumulators; the 32 K block reads are kept LOOKAHEAD ahead of
            // their MFMAs (the compiler's own order kept one or two).
            floatx4 sT[4];
            {
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) sT[kk] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int st = 0; st < 8; ++st)
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk) {
                        const half8 ka = *reinterpret_cast<const half8*>(Kb + (8 * kk + st) * 1024 + 16 * lane);
                        sT[kk] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qf[st], sT[kk], 0, 0, 0);
                    }
                sched_reads_ahead<0>();
            }
            if (kt + 1 < nkt) fetch(kt + 1, b ^ 1, 32);
            // online softmax (base 2); only tiles that reach past the wave's
            // first row need the causal mask
            float mx = -INFINITY;
            if (k0 + KT - 1 > r0) {                 // wave-uniform
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if (k0 + frag_key(kk, 4 * lq + e) > tok) sT[kk][e] = -INFINITY;
                        mx = fmaxf(mx, sT[kk][e]);
                    }
            } else {
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                    for (int e = 0; e < 4; ++e) mx = fmaxf(mx, sT[kk][e]);
            }
            mx = max_xor32(max_xor16(mx));
            // key 0 is visible to every row, so mx is finite from tile 0 on
            const float m_new = mx > m_run + RESCALE_SLACK ? mx : m_run;
            const float corr = __builtin_amdgcn_exp2f(m_run - m_new);      // 1 unless moved; 0 on tile 0
            m_run = m_new;
            half8 pf[2];                            // PV A operand: keys 32 ks + 8 lq .. + 7 of row lr
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    pf[ks][e] = (_Float16)__builtin_amdgcn_exp2f(sT[2 * ks][e] - m_new);
                    pf[ks][4 + e] = (_Float16)__builtin_amdgcn_exp2f(sT[2 * ks + 1][e] - m_new);
                }
            // rescale O (lane (dim lr, lq) holds rows 4lq + e) when any row of
            // the wave moved its reference max
            if (__any(corr != 1.0f)) {
                float f[4];                     // row 4lq + e's factor sits in lane 4lq + e
#pragma unroll
                for (int e = 0; e < 4; ++e) f[e] = __shfl(corr, 4 * lq + e);
#pragma unroll
                for (int dt = 0; dt < 17; ++dt) {
                    O[dt][0] *= f[0]; O[dt][1] *= f[1]; O[dt][2] *= f[2]; O[dt][3] *= f[3];
                }
            }
            // O += P V   (16x16x32; B lane (dim, lq) holds keys 32 ks + 8 lq .. + 7),
            // the V^T block reads LOOKAHEAD ahead of their MFMAs
            {
#pragma unroll
                for (int dt = 0; dt < 16; ++dt)
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) {
                        const half8 vb = *reinterpret_cast<const half8*>(Vb + (2 * dt + ks) * 1024 + 16 * lane);
                        O[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pf[ks], vb, O[dt], 0, 0, 0);
                    }
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) O[16] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pf[ks], ones, O[16], 0, 0, 0);
                sched_reads_ahead<2>();
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // next tile landed (this wave's part)
            __syncthreads();                    // ... for every wave; this tile fully consumed
        }

        // 3. out = (O / l) * sigmoid(gate), bf16 (gemv.rs:1441-1444); O[16][e]
        //    is row 4lq + e's sum of P, in this very lane.  Every gate load is
        //    issued before the first store: the compiler cannot tell the two
        //    pointers apart, and interleaved they cost one memory round trip
        //    per element.
        uint16_t gbuf[4][16];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int tc = min(r0 + 4 * lq + e, A.S - 1);
            const uint16_t* gate = A.q_gate + ((size_t)tc * QM_GQA_HEADS + qh) * (2 * QM_GQA_HD) + QM_GQA_HD + lr;
#pragma unroll
            for (int dt = 0; dt < 16; ++dt) gbuf[e][dt] = gate[16 * dt];
        }
        float iv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) iv[e] = 1.0f / O[16][e];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = r0 + 4 * lq + e;
            if (t >= A.S) continue;
            uint16_t* o = A.out + ((size_t)t * QM_GQA_HEADS + qh) * QM_GQA_HD + lr;
#pragma unroll
            for (int dt = 0; dt < 16; ++dt)
                o[16 * dt] = f32_to_bf16((O[dt][e] * iv[e]) * sigmoid_fast(bf16_to_f32(gbuf[e][dt])));
        }
        if (tid == 0) item_s = claim(home, nxt);
        __syncthreads();
        item = item_s;
    }
}
