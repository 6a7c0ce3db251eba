// dn_decode.hip -- Gated DeltaNet recurrent decode step for gfx950.
//
// Replaces the mixer slice of forward_deltanet_decode (gemv.rs:744-883):
// conv1d+SiLU (layer mode), per-head L2 norm of q/k, alpha/beta gates, the
// delta-rule update of the per-v-head 128x128 fp32 state and the gated
// RMSNorm epilogue.
//
// The state update is a pure HBM stream: each state row S[r,:] (512 B) is
// read once and written once.  One sweep replaces the reference's four
// passes (decay, retrieve, update, output; simd.rs:304-361):
//   Sd = alpha*S; p = Sd.k; delta = beta*(v[r]-p); S' = Sd + delta*k;
//   y[r] = S'.q  (S' is still in registers).
// Layout: a workgroup owns one (sequence, v-head), all 128 rows.  A 16-lane
// DPP row owns one state row at a time; lane l holds columns 4l..4l+3 and
// 64+4l..64+4l+3, so every dwordx4 load of a wave covers four consecutive
// rows contiguously.  Row dot products reduce inside the DPP row (4 DPP
// adds, no LDS).  The head never spans workgroups: publishing rows to
// another workgroup needs an agent-scope fence, i.e. an L2 writeback and
// invalidate, which measured 4-50x slower than the whole update.
#include "qm_device.h"
#include "qm_kernel_args.h"

// gemv.rs:744-772 (layer mode): depthwise causal conv with the old buffer,
// buffer shift, SiLU.  One thread per (sequence, channel), so the in-place
// buffer update has no readers other than its writer.
extern "C" __global__ __launch_bounds__(256) void qm_dn_conv_silu(DnConvArgs A) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)A.batch * QM_DN_QKV_DIM) return;
    const int ch = (int)(idx % QM_DN_QKV_DIM);
    float* buf = A.conv_buf + idx * 3;
    const float4 w = ld4(A.conv_w + ch * 4);
    const float x = A.qkv[idx];
    const float b0 = buf[0], b1 = buf[1], b2 = buf[2];
    A.act[idx] = silu_f(conv_taps4(b0, b1, b2, x, w));
    buf[0] = b1;
    buf[1] = b2;
    buf[2] = x;
}

QM_DEV float dot8(float4 a0, float4 a1, float4 b0, float4 b1) {
    float s = a0.x * b0.x;
    s = fmaf(a0.y, b0.y, s); s = fmaf(a0.z, b0.z, s); s = fmaf(a0.w, b0.w, s);
    s = fmaf(a1.x, b1.x, s); s = fmaf(a1.y, b1.y, s); s = fmaf(a1.z, b1.z, s);
    s = fmaf(a1.w, b1.w, s);
    return s;
}

QM_DEV float4 scale4(float4 a, float s) { return make_float4(a.x * s, a.y * s, a.z * s, a.w * s); }

// gemv.rs:643-649 + :780-785: x /= ||x|| when ||x|| > 1e-12 (per head of 128,
// the 16 lanes of a DPP row hold the whole head), times `scale`.
// 1/||x|| from v_rsq_f32 (1 ulp).
QM_DEV void l2norm_row(float4& x0, float4& x1, float scale) {
    float ss = x0.x * x0.x + x0.y * x0.y + x0.z * x0.z + x0.w * x0.w
             + x1.x * x1.x + x1.y * x1.y + x1.z * x1.z + x1.w * x1.w;
    ss = row_sum16(ss);
    const float inv = (ss > 1e-24f ? __builtin_amdgcn_rsqf(ss) : 1.0f) * scale;
    x0 = scale4(x0, inv);
    x1 = scale4(x1, inv);
}

// The gates on the hardware transcendentals (exp_fast, softplus_fast,
// sigmoid_fast: v_exp_f32 / v_log_f32 / v_rcp_f32, a few ulp from libm):
// every thread of a workgroup evaluates them, and on a 16-lane SIMD each
// wave64 VALU instruction takes 4 cycles, so libm's expansions were a large
// part of a batch-1 step.  gemv.rs:788-800: alpha = exp(-exp(A_log)
// softplus(a + dt_bias)), softplus(x) = x above 20, else ln(1 + e^x);
// beta = sigmoid(b).

template <int RPG>
QM_DEV void dn_decode_body(const DnDecodeArgs& A) {
    constexpr int GROUPS = QM_DN_HD / RPG;       // 16-lane groups per workgroup
    __shared__ float ys[QM_DN_HD];

    const int tid = threadIdx.x;
    const int g = tid >> 4, l = tid & 15;
    const int bid = blockIdx.x;
    const int vh = bid % QM_DN_V_HEADS;
    const int b = bid / QM_DN_V_HEADS;
    const int qkh = vh >> 1;                      // GVA: vh -> vh/2 (gemv.rs:806)

    const float* act = A.act + (size_t)b * QM_DN_QKV_DIM;
    float* S = A.state + (size_t)b * A.state_stride + (size_t)vh * QM_DN_HEAD_ELEMS;

    // q and k first: a wave's loads return in issue order, so their norms
    // (and the gates, from scalar loads) run while the state rows are in
    // flight.  Then the state, the HBM stream: group g owns rows g,
    // g + GROUPS, ...; at each i the groups of a wave cover consecutive
    // rows, so every wave instruction reads contiguous 2 KB.
    float4 q0 = ld4(act + qkh * QM_DN_HD + 4 * l), q1 = ld4(act + qkh * QM_DN_HD + 64 + 4 * l);
    float4 k0 = ld4(act + 2048 + qkh * QM_DN_HD + 4 * l), k1 = ld4(act + 2048 + qkh * QM_DN_HD + 64 + 4 * l);
    float vr[RPG];
#pragma unroll
    for (int i = 0; i < RPG; ++i) vr[i] = act[2 * 2048 + vh * QM_DN_HD + g + GROUPS * i];
    __builtin_amdgcn_sched_barrier(0);           // keep these loads ahead of the state's
    float4 s0[RPG], s1[RPG];
#pragma unroll
    for (int i = 0; i < RPG; ++i) {
        const float* row = S + (size_t)(g + GROUPS * i) * QM_DN_HD;
        s0[i] = ld4(row + 4 * l);
        s1[i] = ld4(row + 64 + 4 * l);
    }
    // The epilogue's inputs (norm weight, z gate) do not depend on the
    // update: fetch them with the state so the norm costs no extra round trip.
    float zz = 0.0f;
    uint32_t nw_bits = 0;                        // converted where it is used, after the update
    if (tid < QM_DN_HD) {
        zz = A.z[(size_t)b * QM_DN_V_DIM + vh * QM_DN_HD + tid];
        nw_bits = A.norm_w[tid];
    }
    const float a_in = A.a[b * QM_DN_V_HEADS + vh], b_in = A.b[b * QM_DN_V_HEADS + vh];
    const float a_log = A.a_log[vh], dt_bias = A.dt_bias[vh];

    l2norm_row(q0, q1, 0.08838834764831845f);    // q *= 1/sqrt(128)
    l2norm_row(k0, k1, 1.0f);

    const float alpha = exp_fast(-exp_fast(a_log) * softplus_fast(a_in + dt_bias));
    const float beta = sigmoid_fast(b_in);

#pragma unroll
    for (int i = 0; i < RPG; ++i) {
        const float4 d0 = scale4(s0[i], alpha), d1 = scale4(s1[i], alpha);
        const float p = row_sum16(dot8(d0, d1, k0, k1));
        const float delta = beta * (vr[i] - p);
        float4 n0, n1;
        n0.x = fmaf(delta, k0.x, d0.x); n0.y = fmaf(delta, k0.y, d0.y);
        n0.z = fmaf(delta, k0.z, d0.z); n0.w = fmaf(delta, k0.w, d0.w);
        n1.x = fmaf(delta, k1.x, d1.x); n1.y = fmaf(delta, k1.y, d1.y);
        n1.z = fmaf(delta, k1.z, d1.z); n1.w = fmaf(delta, k1.w, d1.w);
        float* row = S + (size_t)(g + GROUPS * i) * QM_DN_HD;
        st4(row + 4 * l, n0);
        st4(row + 64 + 4 * l, n1);
        const float y = row_sum16(dot8(n0, n1, q0, q1));
        if (l == 0) ys[g + GROUPS * i] = y;
    }
    __syncthreads();

    // gemv.rs:865-883: per-head RMSNorm (plain gamma, eps 1e-6) * silu(z).
    // Waves 0 and 1 each reduce the 128 squares with the same wave tree, so
    // both hold the same sum (the reference sums rows in order; the
    // difference is a rounding of the sum, ~1e-7 relative).
    if (tid < QM_DN_HD) {
        const int ln = tid & 63;
        const float y0 = ys[ln], y1 = ys[64 + ln];
        const float ss = wave_sum64(fmaf(y1, y1, y0 * y0));
        const float inv_rms = __builtin_amdgcn_rsqf(ss * (1.0f / (float)QM_DN_HD) + 1e-6f);
        asm volatile("" : "+v"(nw_bits));
        const float nw = f16_to_f32((uint16_t)nw_bits);
        A.out[(size_t)b * QM_DN_V_DIM + vh * QM_DN_HD + tid] = ys[tid] * inv_rms * (nw * silu_fast(zz));
    }
}

// One workgroup per (sequence, v-head) holds the whole head, so the norm
// needs no cross-workgroup exchange.  Variants differ only in threads per
// workgroup (rows per 16-lane group 8 / 4 / 2 -> 256 / 512 / 1024 threads).
extern "C" __global__ __launch_bounds__(256) void qm_dn_decode_t256(DnDecodeArgs A) { dn_decode_body<8>(A); }
extern "C" __global__ __launch_bounds__(512) void qm_dn_decode_t512(DnDecodeArgs A) { dn_decode_body<4>(A); }
extern "C" __global__ __launch_bounds__(1024) void qm_dn_decode_t1024(DnDecodeArgs A) { dn_decode_body<2>(A); }
