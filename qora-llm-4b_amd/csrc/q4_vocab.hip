// q4_vocab.hip -- the vocabulary side of a decode step for gfx950: the
// embedding row lookup and the lm_head (tied to the embedding).
//
// The embedding is a Q4Weight with k = vocab rows and n = hidden columns
// (write_embedding_weight, convert.rs:390-415): row v is token v's embedding,
// cut into hidden / 32 groups of 32 columns, each with one f16 scale and 16
// code bytes (low nibble = even column, value = scale * (q - 8)).  Both
// kernels read it in that reference layout, which is already what they want
// (one token's row is contiguous):
//   packed u8 [vocab][hidden/2], scales f16 [vocab][hidden/32].
//
// qm_q4_lm_head: logits[v] = rms_norm(x, final_norm) . row v
// (lm_head_parallel's Q4 arm, gemv.rs:678-708, after the final rms_norm,
// gemv.rs:1074-1076).  248,320 rows x 1,440 bytes = 358 MB per token: an HBM
// stream.
// The RMSNorm is applied by linearity, as in the projection GEMVs:
// logit = inv_rms * (x (1 + gamma)) . row, with inv_rms from the lanes' own
// x slices.  Dequantization: the -8 code offset is applied once per group
// through the group's sum of x, and each code converts with one
// v_cvt_f32_ubyteN.
//
// qm_q4_embed: x[t] = row ids[t] dequantized (embed_lookup_q4,
// gemv.rs:544-563): s * (q - 8) is exact in f32, so rows are bit-identical
// to the reference's.
#include "qm_device.h"
#include "qm_kernel_args.h"

// 8 codes (one 32-bit word: columns 8t .. 8t + 7 of a group) against the
// matching x values; returns sum q * x over them.
QM_DEV float q4_word_dot(uint32_t w, const float* xw, float acc) {
    uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
    // keep the masks: the optimiser would otherwise fold each into a
    // per-nibble bit-field extract
    asm volatile("" : "+v"(lo), "+v"(hi));
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        acc = fmaf((float)((lo >> (8 * b)) & 0xffu), xw[2 * b], acc);
        acc = fmaf((float)((hi >> (8 * b)) & 0xffu), xw[2 * b + 1], acc);
    }
    return acc;
}

// A workgroup has 4 G threads (G = hidden / 32 groups per row; 320 at
// hidden 2560): thread t = G r + g takes group g of row r of every batch of
// four rows, so its 32 values of x, (1 + gamma) applied, stay in registers
// for the whole launch, and a batch is one 16-byte code load and one scale
// per thread.  G % 16 == 0, so each 16-lane DPP row of a wave lies inside
// one row of the batch: its partial sum goes to LDS, and after LMH_SB
// batches one thread per row adds the row's G / 16 partials in a fixed
// order.  Workgroups stride over these super-batches of 4 LMH_SB rows.
#define LMH_SB 8
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

extern "C" __global__ __launch_bounds__(1024) void qm_q4_lm_head(LmHeadArgs A) {
    __shared__ float part[LMH_SB][64];          // [batch][16-lane segment]
    __shared__ float red[16];
    const int t = threadIdx.x, K = A.k, G = K / 32;
    const int r = t / G, g = t % G, seg = t >> 4, sl = t & 15;

    float xs[32];
    {
        const float4* xp = reinterpret_cast<const float4*>(A.x + 32 * g);
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            const float4 q = xp[v];
            xs[4 * v] = q.x;
            xs[4 * v + 1] = q.y;
            xs[4 * v + 2] = q.z;
            xs[4 * v + 3] = q.w;
        }
    }
    float inv = 1.0f;
    if (A.norm_w) {
        // gemv.rs:572-574 over row 0's threads, which hold all of x
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < 32; ++e) ss = fmaf(xs[e], xs[e], ss);
        ss = row_sum16(ss);
        if (r == 0 && sl == 0) red[seg] = ss;
        const uint4* gp = reinterpret_cast<const uint4*>(A.norm_w + 32 * g);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint4 q = gp[v];
            const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                xs[8 * v + 2 * h] *= 1.0f + f16_to_f32((uint16_t)(wd[h] & 0xffffu));
                xs[8 * v + 2 * h + 1] *= 1.0f + f16_to_f32((uint16_t)(wd[h] >> 16));
            }
        }
        __syncthreads();
        float tot = 0.0f;
        for (int i = 0; i < G / 16; ++i) tot += red[i];
        inv = 1.0f / sqrtf(tot / (float)K + 1e-6f);
    }
    float sx = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; ++e) sx += xs[e];
    sx *= 8.0f;

    const int nsb = (A.vocab + 4 * LMH_SB - 1) / (4 * LMH_SB);
    const size_t rstride = (size_t)(K / 2);
    for (int sb = blockIdx.x; sb < nsb; sb += gridDim.x) {
        u32x4 c[LMH_SB];
        uint16_t sc[LMH_SB];
#pragma unroll
        for (int b = 0; b < LMH_SB; ++b) {
            const size_t row = (size_t)min((sb * LMH_SB + b) * 4 + r, A.vocab - 1);
            // read once per token: non-temporal, so the stream does not evict x
            c[b] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(A.codes + row * rstride + 16 * g));
            sc[b] = A.scales[row * G + g];
        }
#pragma unroll
        for (int b = 0; b < LMH_SB; ++b) {
            float d = 0.0f;
            d = q4_word_dot(c[b].x, &xs[0], d);
            d = q4_word_dot(c[b].y, &xs[8], d);
            d = q4_word_dot(c[b].z, &xs[16], d);
            d = q4_word_dot(c[b].w, &xs[24], d);
            const float p = row_sum16(f16_to_f32(sc[b]) * (d - sx));
            if (sl == 0) part[b][seg] = p;
        }
        __syncthreads();
        if (t < 4 * LMH_SB) {
            const int b = t >> 2, rr = t & 3;
            const int row = (sb * LMH_SB + b) * 4 + rr;
            float tot = 0.0f;
            for (int i = 0; i < G / 16; ++i) tot += part[b][rr * (G / 16) + i];
            if (row < A.vocab) A.logits[row] = inv * tot;
        }
        __syncthreads();
    }
}

// One workgroup (64 threads) per token; thread t writes the 32 columns of
// group t, t + 64, ...  An id outside the vocabulary (a slice-index panic in
// the reference) writes a row of NaN.
extern "C" __global__ __launch_bounds__(64) void qm_q4_embed(EmbedArgs A) {
    const int t = blockIdx.x, tid = threadIdx.x;
    const int id = A.ids[t];
    const int K = A.k, GPR = K / 32;
    float* out = A.out + (size_t)t * K;
    const bool ok = id >= 0 && id < A.vocab;
    const size_t row = ok ? (size_t)id : 0;
    for (int g = tid; g < GPR; g += 64) {
        const uint4 c = *reinterpret_cast<const uint4*>(A.codes + row * (size_t)(K / 2) + 16 * g);
        const float s = ok ? f16_to_f32(A.scales[row * GPR + g]) : __builtin_nanf("");
        const uint32_t wd[4] = {c.x, c.y, c.z, c.w};
        float v[32];
#pragma unroll
        for (int h = 0; h < 4; ++h)
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const uint32_t byte = (wd[h] >> (8 * b)) & 0xffu;
                v[8 * h + 2 * b] = s * (float)((int)(byte & 0x0fu) - 8);
                v[8 * h + 2 * b + 1] = s * (float)((int)(byte >> 4) - 8);
            }
        float4* o = reinterpret_cast<float4*>(out + 32 * g);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = make_float4(v[4 * e], v[4 * e + 1], v[4 * e + 2], v[4 * e + 3]);
    }
}
