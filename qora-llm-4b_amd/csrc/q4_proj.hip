// q4_proj.hip -- Q4 projections (the GEMVs around the token mixer) for gfx950.
//
// A Q4Weight (gemv.rs:29-34) maps k inputs to n outputs.  Each input row is
// cut into groups of 32 output columns with one f16 scale (absmax / 7) and 16
// bytes of 4-bit codes q, value = scale * (q - 8); byte j of a group holds
// column 2j in its low nibble and 2j + 1 in its high nibble (quantize_q4,
// convert.rs:437-467).  The reference stores it row-major:
//   packed u8 [k][n/2], scales f16 [k][n/32].
// On the device a weight is kept tile-major (qm_q4_repack, once at load
// time, as the reference's wgpu loader repacks for its backend,
// gpu_loader.rs:82-106): column tiles of T = 16 columns (T = 8 when
// n < 4096, so that even a 2560-wide weight spreads over 320 workgroups),
//   codes u8 [n/T][k][T/2], gscales f16 [n/32][k],
// so that everything one output tile needs is one contiguous stream.
//
// qm_q4_gemv computes y = x W (gemv_q4, gemv.rs:451-467, inner loop
// :412-445) for one input row, for up to four weights that share x in one
// launch (a launch costs a few microseconds of fixed time, about what a
// 2560x4096 weight takes to stream).  Optional fusions, each what the
// reference does right around that gemv call:
//   - x <- rms_norm(x, gamma) first (1 + gamma, eps 1e-6; gemv.rs:571-579),
//     as before in_proj_* / q,k,v_proj and before the MLP (gemv.rs:740,893);
//   - y <- residual + x W (the residual adds after out_proj / o_proj and
//     down_proj, gemv.rs:889-890,896);
//   - qm_q4_gate_up: silu(x Wg) * (x Wu) for one tile of both weights per
//     workgroup (fused_gate_up_q4, gemv.rs:469-526);
//   - on the first weight, the DeltaNet conv1d step + SiLU (gemv.rs:744-772)
//     of the in_proj_qkv output, with its conv buffer shifted in place.
// One workgroup owns one column tile and all k rows, so the result needs
// no second pass: lane t takes rows t, t + 512, ..., and loads its 8 rows'
// codes, scales, x (and norm weights) before any arithmetic, at clamped
// rows so that no load waits behind a branch.  The T partial sums of every
// lane are reduced across the wave in registers (a transpose-reduce over
// lane swaps), then across the waves through LDS behind one barrier, in a
// fixed order (bit-reproducible run to run).  Dequantization costs ~2.4 VALU ops per weight: the codes are split
// into low and high nibble bytes by two masks, each byte converts with one
// v_cvt_f32_ubyteN, and the fma uses q itself, the -8 offset being applied
// once per lane through sum(scale * x).  The RMSNorm is applied by
// linearity: y = inv_rms * (x (1 + gamma)) W, so its sum of squares comes
// from the same x loads and the factor scales the column sums.
#include "qm_device.h"
#include "qm_kernel_args.h"

#define Q4_THREADS 512
#define Q4_STEPS 8          // rows per lane in flight

template <int T> struct Q4Codes;                          // T/2 bytes of codes
template <> struct Q4Codes<16> { typedef uint2 type; };
template <> struct Q4Codes<8> { typedef uint32_t type; };
template <int T> struct Q4Pair;                           // two consecutive rows' codes
template <> struct Q4Pair<16> {
    typedef uint4 type;
    static QM_DEV uint2 half(uint4 v, int h) { return h ? make_uint2(v.z, v.w) : make_uint2(v.x, v.y); }
};
template <> struct Q4Pair<8> {
    typedef uint2 type;
    static QM_DEV uint32_t half(uint2 v, int h) { return h ? v.y : v.x; }
};

QM_DEV void q4_word(float* acc, uint32_t w, float sx) {  // 8 codes: columns 0..7 of acc
    uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
    // opaque to the optimiser, which would otherwise fold each mask into a
    // per-nibble bit-field extract (one more op each)
    asm volatile("" : "+v"(lo), "+v"(hi));
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        acc[2 * b] = fmaf((float)((lo >> (8 * b)) & 0xffu), sx, acc[2 * b]);
        acc[2 * b + 1] = fmaf((float)((hi >> (8 * b)) & 0xffu), sx, acc[2 * b + 1]);
    }
}
QM_DEV void q4_accumulate(float (&acc)[16], uint2 c, float sx) { q4_word(acc, c.x, sx); q4_word(acc + 8, c.y, sx); }
QM_DEV void q4_accumulate(float (&acc)[8], uint32_t c, float sx) { q4_word(acc, c, sx); }

// Wave-level sum of each of a lane's T column partials by transpose-reduce:
// each step pairs lane l with l ^ 32, ^16, ^8 (and ^4 for T = 16), and each
// lane keeps the half of its columns its side of the pair owns, summed with
// the partner's copy of them; then the remaining lane bits are summed.  At
// the end lane l holds the wave's total of column q4_col<T>(l) (the same in
// the 64 / T lanes that share it).  No LDS, no barrier; a fixed order, so
// the result is reproducible run to run.
QM_DEV float xor_swz4(float x) {            // the value of lane l ^ 4 (ds_swizzle bit mode)
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), 0x101F));
}
// (n is a template parameter: as a runtime argument the compiler did not
// unroll these loops and indexed v through 16-way compare/select chains)
template <int N>
QM_DEV void halve32(float* v) {             // N values -> N/2: lanes < 32 keep 0..N/2-1
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[j]), __float_as_uint(v[j + N / 2]), false, false);
        v[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
}
template <int N>
QM_DEV void halve16(float* v) {             // even 16-lane rows keep 0..N/2-1
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[j]), __float_as_uint(v[j + N / 2]), false, false);
        v[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
}
template <int BIT, int N>
QM_DEV void halve_dpp(float* v, int lane) {  // lanes with bit BIT clear keep 0..N/2-1
    const bool hi = (lane >> BIT) & 1;
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
        const float keep = hi ? v[j + N / 2] : v[j];
        const float send = hi ? v[j] : v[j + N / 2];
        const float got = BIT == 3 ? dpp_f32<0x128>(send) : xor_swz4(send);   // row_ror:8 = lane ^ 8
        v[j] = keep + got;
    }
}
template <int T> QM_DEV int q4_col(int lane) {
    return T == 16 ? 8 * ((lane >> 5) & 1) + 4 * ((lane >> 4) & 1) + 2 * ((lane >> 3) & 1) + ((lane >> 2) & 1)
                   : 4 * ((lane >> 5) & 1) + 2 * ((lane >> 4) & 1) + ((lane >> 3) & 1);
}
template <int T>
QM_DEV float q4_wave_reduce(float (&v)[T], int lane) {
    halve32<T>(v);
    halve16<T / 2>(v);
    halve_dpp<3, T / 4>(v, lane);
    float x;
    if (T == 16) {
        halve_dpp<2, 2>(v, lane);
        x = v[0];
    } else {
        x = v[0];
        x += xor_swz4(x);
    }
    x += dpp_f32<0x4E>(x);                  // lane ^ 2
    x += dpp_f32<0xB1>(x);                  // lane ^ 1
    return x;
}

// base[idx] with a 32-bit byte offset from a wave-uniform base, so the load
// takes the scalar-base + 32-bit vector-offset form (no 64-bit address
// arithmetic per lane)
template <class V>
QM_DEV V ld_off(const V* base, uint32_t idx) {
    return *reinterpret_cast<const V*>(reinterpret_cast<const char*>(base) + (size_t)(idx * (uint32_t)sizeof(V)));
}

template <bool GATE_UP, bool PAIR, bool NORM, int T, int STEPS, int THREADS>
QM_DEV void q4_tile(const Q4GemvArgs& A, int p, int tile, float (*red)[33]) {
    typedef typename Q4Codes<T>::type CodeT;
    const int tid = threadIdx.x;
    const int K = A.k;
    const int g = tile / (32 / T);                        // the tile's 32-column scale group
    const CodeT* codes = reinterpret_cast<const CodeT*>(A.codes[p]) + (size_t)tile * K;
    const uint16_t* gsc = A.gscales[p] + (size_t)g * K;
    const CodeT* codes_u = GATE_UP ? reinterpret_cast<const CodeT*>(A.codes[1]) + (size_t)tile * K : nullptr;
    const uint16_t* gsc_u = GATE_UP ? A.gscales[1] + (size_t)g * K : nullptr;
    // NORM (A.norm_w set, uniform over the launch) is a template parameter: a
    // load under a condition would wait for its data before the next step's
    // loads issue
    const uint16_t* nwp = A.norm_w;

    float acc[T], acc_u[GATE_UP ? T : 1];
#pragma unroll
    for (int j = 0; j < T; ++j) acc[j] = 0.0f;
#pragma unroll
    for (int j = 0; j < (GATE_UP ? T : 1); ++j) acc_u[j] = 0.0f;
    float bsum = 0.0f, bsum_u = 0.0f, ss = 0.0f;
    if (PAIR) {
        // two consecutive rows per load: their codes (2 x T/2 bytes), scales,
        // x values and norm weights are adjacent, so one load instruction of
        // twice the width takes both (k is even on this path)
        typedef typename Q4Pair<T>::type PairT;
        const int KP = K >> 1;
        const PairT* codes2 = reinterpret_cast<const PairT*>(codes);
        const PairT* codes2_u = reinterpret_cast<const PairT*>(codes_u);
        const uint32_t* gsc2 = reinterpret_cast<const uint32_t*>(gsc);
        const uint32_t* gsc2_u = reinterpret_cast<const uint32_t*>(gsc_u);
        const uint32_t* nwp2 = reinterpret_cast<const uint32_t*>(nwp);
        const float2* x2 = reinterpret_cast<const float2*>(A.x);
        constexpr int PS = STEPS / 2;
        for (int k0 = 0; k0 < KP; k0 += THREADS * PS) {
            PairT pk[PS], pu[GATE_UP ? PS : 1];
            uint32_t sc[PS], su[GATE_UP ? PS : 1], nw[PS];
            float2 xv[PS];
#pragma unroll
            for (int s = 0; s < PS; ++s) {
                const uint32_t kp = min((uint32_t)(k0 + tid + THREADS * s), (uint32_t)(KP - 1));
                pk[s] = ld_off(codes2, kp);
                sc[s] = ld_off(gsc2, kp);
                if (GATE_UP) {
                    pu[s] = ld_off(codes2_u, kp);
                    su[s] = ld_off(gsc2_u, kp);
                }
                xv[s] = ld_off(x2, kp);
                if (NORM) nw[s] = ld_off(nwp2, kp);
            }
            const bool full = k0 + THREADS * PS <= KP;
#pragma unroll
            for (int s = 0; s < PS; ++s) {
                if (!full && k0 + THREADS * s + (tid & ~63) >= KP) break;
                const bool ok = full || k0 + tid + THREADS * s < KP;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const float xl = ok ? (h ? xv[s].y : xv[s].x) : 0.0f;
                    ss = fmaf(xl, xl, ss);
                    const float xn = NORM ? xl * (1.0f + f16_to_f32((uint16_t)(nw[s] >> (16 * h)))) : xl;
                    const float sx = f16_to_f32((uint16_t)(sc[s] >> (16 * h))) * xn;
                    bsum += sx;
                    q4_accumulate(acc, Q4Pair<T>::half(pk[s], h), sx);
                    if (GATE_UP) {
                        const float sxu = f16_to_f32((uint16_t)(su[s] >> (16 * h))) * xn;
                        bsum_u += sxu;
                        q4_accumulate(reinterpret_cast<float(&)[T]>(acc_u), Q4Pair<T>::half(pu[s], h), sxu);
                    }
                }
            }
        }
    } else {
        for (int k0 = 0; k0 < K; k0 += THREADS * STEPS) {
            CodeT pk[STEPS], pu[GATE_UP ? STEPS : 1];
            uint16_t sc[STEPS], su[GATE_UP ? STEPS : 1], nw[STEPS];
            float xv[STEPS];
    #pragma unroll
            for (int s = 0; s < STEPS; ++s) {
                const uint32_t k = min((uint32_t)(k0 + tid + THREADS * s), (uint32_t)(K - 1));
                pk[s] = ld_off(codes, k);
                sc[s] = ld_off(gsc, k);
                if (GATE_UP) {
                    pu[s] = ld_off(codes_u, k);
                    su[s] = ld_off(gsc_u, k);
                }
                xv[s] = ld_off(A.x, k);
                if (NORM) nw[s] = ld_off(nwp, k);
            }
            const bool full = k0 + THREADS * STEPS <= K;    // workgroup-uniform: every row valid
    #pragma unroll
            for (int s = 0; s < STEPS; ++s) {
                // rows past k (wave-uniform except in the last wave) add nothing
                if (!full && k0 + THREADS * s + (tid & ~63) >= K) break;
                const float xl = full || k0 + tid + THREADS * s < K ? xv[s] : 0.0f;
                ss = fmaf(xl, xl, ss);
                const float xn = NORM ? xl * (1.0f + f16_to_f32(nw[s])) : xl;   // gemv.rs:575 but inv_rms
                const float sx = f16_to_f32(sc[s]) * xn;                           // gemv.rs:429: scale * x_k
                bsum += sx;
                q4_accumulate(acc, pk[s], sx);
                if (GATE_UP) {
                    const float sxu = f16_to_f32(su[s]) * xn;
                    bsum_u += sxu;
                    q4_accumulate(reinterpret_cast<float(&)[T]>(acc_u), pu[s], sxu);
                }
            }
        }
    }

    // Column sums: each wave reduces its lanes' partials in registers (the
    // -8 code offset applied through the scale * x sums), writes one value
    // per column, and after one barrier thread j < T adds the THREADS / 64
    // waves' values in order.  x's sum of squares for the RMSNorm rides along.
    const int lane = tid & 63, wv = tid >> 6;
#pragma unroll
    for (int j = 0; j < T; ++j) acc[j] = fmaf(-8.0f, bsum, acc[j]);
    const float cs = q4_wave_reduce<T>(acc, lane);
    float cs_u = 0.0f;
    if (GATE_UP) {
#pragma unroll
        for (int j = 0; j < T; ++j) acc_u[j] = fmaf(-8.0f, bsum_u, acc_u[j]);
        cs_u = q4_wave_reduce<T>(reinterpret_cast<float(&)[T]>(acc_u), lane);
    }
    const float ssw = NORM ? wave_sum64(ss) : 0.0f;
    if ((lane & (64 / T - 1)) == 0) {
        red[wv][q4_col<T>(lane)] = cs;
        if (GATE_UP) red[wv][16 + q4_col<T>(lane)] = cs_u;
    }
    if (lane == 0) red[wv][32] = ssw;
    __syncthreads();
    float y = 0.0f, u = 0.0f, sst = 0.0f;
    if (tid < T) {
#pragma unroll
        for (int w = 0; w < THREADS / 64; ++w) {
            y += red[w][tid];
            if (GATE_UP) u += red[w][16 + tid];
            sst += red[w][32];
        }
    }
    // gemv.rs:573: 1 / sqrt(mean(x^2) + 1e-6)
    const float inv = NORM ? 1.0f / sqrtf(sst / (float)K + 1e-6f) : 1.0f;
    y *= inv;
    if (GATE_UP) {
        u *= inv;
        // gemv.rs:524: (g / (1 + exp(-g))) * u
        if (tid < T) A.y[0][T * (size_t)tile + tid] = (y / (1.0f + expf(-y))) * u;
    } else if (tid < T) {
        const size_t c = T * (size_t)tile + tid;
        float v = A.residual[p] ? A.residual[p][c] + y : y;
        if (p == 0 && A.conv_buf) {
            // gemv.rs:744-772 on the in_proj_qkv output: causal depthwise
            // conv over the buffer (oldest .. newest) and v, buffer shift,
            // SiLU
            float* buf = A.conv_buf + c * 3;
            const float4 w = *reinterpret_cast<const float4*>(A.conv_w + c * 4);
            const float b0 = buf[0], b1 = buf[1], b2 = buf[2];
            const float s = conv_taps4(b0, b1, b2, v, w);
            buf[0] = b1;
            buf[1] = b2;
            buf[2] = v;
            v = silu_f(s);
        }
        A.y[p][c] = v;
    }
}

template <bool GATE_UP, bool NORM, int STEPS, int THREADS>
QM_DEV void q4_tile_pick(const Q4GemvArgs& A, int p, int tile, float (*red)[33]) {
    if (A.k & 1) {
        if (A.tile[p] == 16) q4_tile<GATE_UP, false, NORM, 16, STEPS, THREADS>(A, p, tile, red);
        else q4_tile<GATE_UP, false, NORM, 8, STEPS, THREADS>(A, p, tile, red);
    } else {
        if (A.tile[p] == 16) q4_tile<GATE_UP, true, NORM, 16, STEPS, THREADS>(A, p, tile, red);
        else q4_tile<GATE_UP, true, NORM, 8, STEPS, THREADS>(A, p, tile, red);
    }
}

template <bool GATE_UP, int STEPS, int THREADS, bool WITH_NORM = true>
QM_DEV void q4_gemv_body(const Q4GemvArgs& A) {
    __shared__ float red[THREADS / 64][33];   // per wave: column sums (gate, up), x's sum of squares
    // which weight: workgroups wstart[p] .. wstart[p+1]-1 are weight p's
    // tiles (gate / up: weights 0 and 1 share the tile index)
    int p = 0;
    if (!GATE_UP) {
#pragma unroll
        for (int q = 1; q < QM_Q4_MAX_OUT; ++q)
            if (q < A.count && (int)blockIdx.x >= A.wstart[q]) p = q;
    }
    const int tile = (int)blockIdx.x - A.wstart[p];
    if (WITH_NORM && A.norm_w) q4_tile_pick<GATE_UP, WITH_NORM, STEPS, THREADS>(A, p, tile, red);
    else q4_tile_pick<GATE_UP, false, STEPS, THREADS>(A, p, tile, red);
}

extern "C" __global__ __launch_bounds__(Q4_THREADS) void qm_q4_gemv(Q4GemvArgs A) {
    q4_gemv_body<false, Q4_STEPS, Q4_THREADS>(A);
}

// 256 threads, 10 rows (5 row pairs) per lane: one load round at k = 2560,
// and at 132 VGPRs three workgroups per CU, so the 576 tiles of the 2560 x
// 9216 gate / up pair are resident in one dispatch round (the 512-thread form
// fitted two per CU and ran 3% slower per model token).
extern "C" __global__ __launch_bounds__(256) void qm_q4_gate_up(Q4GemvArgs A) {
    q4_gemv_body<true, 10, 256>(A);
}

// Shape-fitted forms.  A launch's workgroups should all be resident at once
// (a second dispatch round repeats the whole load -> reduce latency), and a
// lane's rows should come in as few load rounds as possible:
//   k <= 2560 (the hidden size): 256 threads of 10 rows, one load round, 84
//     VGPRs (five workgroups per CU, 1280 slots for the 776 tiles of the
//     fused DeltaNet input projections);
//   k <= 9216 without a norm (the MLP's down_proj): 18 rows per lane, one
//     load round, 115 VGPRs (two workgroups per CU, 512 slots for 320
//     tiles); the host sends a launch with a norm to the general form.
// (512-thread forms of 5 rows for k <= 2560, of 18 or 12 rows at 256 threads
// for down_proj, and of 16 at 256 threads for the general case all measured
// slower over a model token.)
extern "C" __global__ __launch_bounds__(256)
void qm_q4_gemv_hidden(Q4GemvArgs A) {
    q4_gemv_body<false, 10, 256>(A);
}
extern "C" __global__ __launch_bounds__(Q4_THREADS) __attribute__((amdgpu_waves_per_eu(4)))
void qm_q4_gemv_inter(Q4GemvArgs A) {
    q4_gemv_body<false, 18, Q4_THREADS, false>(A);
}

// Reference layout -> tile-major.  Workgroup = 64 rows x 16 groups: each
// thread reads one 16-byte group block and one scale (consecutive along a
// row), and writes the block's 32 / T tile slices (consecutive along k
// within a tile: 64 rows x T/2 bytes).
extern "C" __global__ __launch_bounds__(256) void qm_q4_repack(Q4RepackArgs A) {
    __shared__ uint4 tc[16][65];
    __shared__ uint16_t ts[16][66];
    const int tid = threadIdx.x;
    const int G = A.n / 32, T = A.tile;
    const int gb = blockIdx.x % ((G + 15) / 16), kb = blockIdx.x / ((G + 15) / 16);
    const int k0 = kb * 64, g0 = gb * 16;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const int r = p * 16 + (tid >> 4), j = tid & 15;
        const int k = k0 + r, g = g0 + j;
        if (k < A.k && g < G) {
            tc[j][r] = *reinterpret_cast<const uint4*>(A.packed + (size_t)k * (A.n / 2) + 16 * (size_t)g);
            ts[j][r] = A.scales[(size_t)k * G + g];
        }
    }
    __syncthreads();
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const int j = p * 4 + (tid >> 6), r = tid & 63;
        const int k = k0 + r, g = g0 + j;
        if (k < A.k && g < G) {
            const uint4 v = tc[j][r];
            if (T == 16) {
                uint2* dst = reinterpret_cast<uint2*>(A.codes);
                dst[(size_t)(2 * g) * A.k + k] = make_uint2(v.x, v.y);
                dst[(size_t)(2 * g + 1) * A.k + k] = make_uint2(v.z, v.w);
            } else {
                uint32_t* dst = reinterpret_cast<uint32_t*>(A.codes);
                dst[(size_t)(4 * g) * A.k + k] = v.x;
                dst[(size_t)(4 * g + 1) * A.k + k] = v.y;
                dst[(size_t)(4 * g + 2) * A.k + k] = v.z;
                dst[(size_t)(4 * g + 3) * A.k + k] = v.w;
            }
            A.gscales[(size_t)g * A.k + k] = ts[j][r];
        }
    }
}

// ---------------------------------------------------------------------------
// Prefill: C[m][n] = X[m][k] W on MFMA (gemm_q4, gemv.rs:529-542, for
// seq_len > 1).  X is f16 (qm_rms_norm_f16 produces it from the f32 hidden
// state, fusing the layer's RMSNorm) or bf16 (the mixer outputs and the
// MLP's silu(g) * u).  W stays Q4 in HBM and is dequantized on its way into
// LDS: s * (q - 8) rounded once to f16 and, for a bf16 X, on to bf16.  An
// f16 X runs v_mfma_f32_16x16x32_f16; a bf16 X is staged as it is and runs
// v_mfma_f32_16x16x32_bf16, so it keeps fp32's range.
// Workgroup tile 128 x 256, four waves of 64 x 128 (4 x 8 MFMA tiles: 12
// fragment reads feed 32 MFMAs), k steps of 32 in two LDS stages with one
// barrier per step.  LDS rows are k-contiguous, X as [m][k] and W as [n][k],
// padded to 40 halves (80 bytes) so the 16 rows of a fragment read land in
// 16 distinct bank slots; a lane's A operand (row m, k 8kg .. +7) and B
// operand (column n, k 8kg .. +7) are then one 16-byte read each.
// ---------------------------------------------------------------------------
#define GM_TK 32
#define GM_LDK 40

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// An f16 pair as a bf16 pair, each rounded to nearest even (the f16 values
// are exact in fp32, so this is one rounding of each).
__device__ __forceinline__ uint32_t f16x2_to_bf16x2(half2 h) {
    const bf16x2 b = bf16x2{(__bf16)(float)h[0], (__bf16)(float)h[1]};
    return __builtin_bit_cast(uint32_t, b);
}

// XBF16: x is bf16 and W is rounded on to bf16 (bf16 MFMA); else both f16.
// GU: the gate/up form.  The workgroup's 256 W rows of LDS are then
// 16-column fragments of the gate and up weights alternately, over 128
// output columns, so a wave's fragments j (gate) and j + 1 (up) hold the
// same outputs and the epilogue writes silu(g) * u as bf16 (whose range,
// unlike f16's, holds any product of the fp32 accumulators).
// A workgroup is WM x WN waves; a wave computes MI x NJ MFMA tiles of
// 16 x 16 (16 MI rows, 16 NJ columns), so the workgroup tile is TM x TN =
// 16 MI WM x 16 NJ WN.  128 x 256 (2 x 2 waves of 64 x 128) where there are
// tiles enough for two workgroups per CU; for narrow outputs that would
// leave CUs idle, 128 x 128 (n = 2560: 10 column tiles of 256) or 64 x 128
// (n = 1024); n = 32 has a kernel of its own below.  The W tile is staged by
// threads 0 .. TN-1.  (64 x 256 tiles, four waves of 64 x 64 side by side,
// measured 2% slower on the 4096-token prefill.)
template <bool XBF16, bool GU, int WM, int WN, int MI, int NJ>
__device__ __forceinline__ void q4_gemm_body(const Q4GemmArgs& A) {
    constexpr int TM = 16 * MI * WM, TN = 16 * NJ * WN, NTH = 64 * WM * WN;
    static_assert(!GU || (WN == 2 && NJ == 8), "the gate/up form pairs fragments j, j + 1 over 256 LDS rows");
    static_assert(NTH >= TN && (TM * GM_TK / NTH == 8 || TM * GM_TK / NTH == 16), "staging shape");
    __shared__ __attribute__((aligned(16))) _Float16 sA[2][TM][GM_LDK];
    __shared__ __attribute__((aligned(16))) _Float16 sB[2][TN][GM_LDK];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    constexpr int NCOLS = GU ? TN / 2 : TN;              // output columns per workgroup
    const int nbn = (A.n + NCOLS - 1) / NCOLS;
    // consecutive workgroups walk n within one row block: the row block's X
    // (k x TM halves) is reused from L2 across its column tiles
    const int bm = (int)blockIdx.x / nbn, bn = (int)blockIdx.x % nbn;
    const int m0 = bm * TM, n0 = bn * NCOLS;
    const int wm = w / WN, wn = w % WN;
    const int T = A.tile, K = A.k;
    const int nk = K / GM_TK;

    // X staging: thread -> row tid / (32 / XH), XH halves of k
    constexpr int XH = TM * GM_TK / NTH;                 // 16 or 8 halves per thread
    const int ar = tid / (32 / XH), ah = tid % (32 / XH);
    const uint16_t* xrow = A.x + (size_t)min(m0 + ar, A.m - 1) * K + XH * ah;
    // W staging: thread -> 8-column block c8 of the tile and RQ rows
    // RQ rq .. +RQ-1 of the step, with every thread taking a share (RQ = 4
    // when the tile has as many columns as the workgroup threads, else 2); a
    // block is 4 code bytes of one row (T = 16: half of a tile row, T = 8: a
    // whole one)
    constexpr int RQ = NTH == TN ? 4 : 2;
    const int c8 = tid / (32 / RQ), rq = tid % (32 / RQ);
    // GU: LDS rows 8 c8 .. +7 are half of fragment c8 / 2, of the up weight
    // when that fragment is odd
    const bool up = GU && ((c8 >> 1) & 1);
    const int ccol = GU ? 16 * (c8 >> 2) + 8 * (c8 & 1) : 8 * c8;
    const int ncl = min(n0 + ccol, A.n - 8);            // valid block for loads
    const size_t cstride = (size_t)(T / 2);
    const uint8_t* bcodes = (up ? A.codes2 : A.codes) + (size_t)(ncl / T) * K * cstride + (ncl % T) / 2 +
                            RQ * rq * cstride;
    const uint16_t* bsc = (up ? A.gscales2 : A.gscales) + (size_t)(ncl / 32) * K + RQ * rq;
    const bool wthread = NTH * RQ == 4 * TN || tid < TN * 4 / RQ;

    // the f16 exponent pattern 0x6400 (1024) of each half, held in a VGPR so
    // that masking a nibble pair into it is one v_and_or_b32 (the mask is
    // the instruction's one literal)
    uint32_t vmagic;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(vmagic));
    uint4 ra0, ra1;
    uint32_t rb[4];
    uint2 rs;                                            // RQ f16 scales of rows RQ rq .. +RQ-1
#define GM_GLOAD(kt)                                                                   \
    do {                                                                               \
        const int k0_ = (kt) * GM_TK;                                                  \
        ra0 = *reinterpret_cast<const uint4*>(xrow + k0_);                            \
        if (XH == 16) ra1 = *reinterpret_cast<const uint4*>(xrow + k0_ + 8);          \
        if (wthread) {                                                                 \
            _Pragma("unroll") for (int i_ = 0; i_ < RQ; ++i_)                          \
                rb[i_] = *reinterpret_cast<const uint32_t*>(bcodes + (size_t)(k0_ + i_) * cstride); \
            if (RQ == 4) rs = *reinterpret_cast<const uint2*>(bsc + k0_);             \
            else rs.x = *reinterpret_cast<const uint32_t*>(bsc + k0_);                \
        }                                                                              \
    } while (0)
    // Columns 2b, 2b + 1 of a row pair come from byte b of each row's block.
    // v_perm_b32 puts the first row's byte at bits 0-7 and the second's at
    // bits 16-23 (of the words, and of the words shifted down by 4 for the
    // high nibbles); masking a nibble pair into 0x6400 | q gives the f16 pair
    // (1024 + q), and packed f16 ops make it s * (q - 8): exact, then one
    // rounding of the product (the same bits as rounding s * (q - 8) from
    // fp32).  Column n's four (two) rows are one 8-byte (4-byte) store.
#define GM_BPAIR(v) (XBF16 ? f16x2_to_bf16x2(v) : __builtin_bit_cast(uint32_t, v))
#define GM_LSTORE(buf)                                                                 \
    do {                                                                               \
        *reinterpret_cast<uint4*>(&sA[buf][ar][XH * ah]) = ra0;                        \
        if (XH == 16) *reinterpret_cast<uint4*>(&sA[buf][ar][XH * ah + 8]) = ra1;      \
        const half2 s01 = __builtin_bit_cast(half2, rs.x), s23 = __builtin_bit_cast(half2, rs.y); \
        uint32_t rh[RQ];                                  /* high nibbles moved down once */ \
        _Pragma("unroll") for (int i_ = 0; i_ < RQ; ++i_) rh[i_] = rb[i_] >> 4;       \
        if (wthread) _Pragma("unroll") for (int b_ = 0; b_ < 4; ++b_) {                \
            const uint32_t sel = 0x0c040c00u + 0x00010001u * b_;                       \
            const half2 k1032 = half2{1032.0f16, 1032.0f16};                           \
            const uint32_t p01 = __builtin_amdgcn_perm(rb[1], rb[0], sel);             \
            const uint32_t q01 = __builtin_amdgcn_perm(rh[1], rh[0], sel);             \
            const half2 l01 = (__builtin_bit_cast(half2, (p01 & 0x000f000fu) | vmagic) - k1032) * s01; \
            const half2 h01 = (__builtin_bit_cast(half2, (q01 & 0x000f000fu) | vmagic) - k1032) * s01; \
            if constexpr (RQ == 4) {                                                   \
                const uint32_t p23 = __builtin_amdgcn_perm(rb[3], rb[2], sel);         \
                const uint32_t q23 = __builtin_amdgcn_perm(rh[3], rh[2], sel);         \
                const half2 l23 = (__builtin_bit_cast(half2, (p23 & 0x000f000fu) | vmagic) - k1032) * s23; \
                const half2 h23 = (__builtin_bit_cast(half2, (q23 & 0x000f000fu) | vmagic) - k1032) * s23; \
                *reinterpret_cast<uint2*>(&sB[buf][8 * c8 + 2 * b_][4 * rq]) = make_uint2(GM_BPAIR(l01), GM_BPAIR(l23)); \
                *reinterpret_cast<uint2*>(&sB[buf][8 * c8 + 2 * b_ + 1][4 * rq]) = make_uint2(GM_BPAIR(h01), GM_BPAIR(h23)); \
            } else {                                                                   \
                *reinterpret_cast<uint32_t*>(&sB[buf][8 * c8 + 2 * b_][2 * rq]) = GM_BPAIR(l01); \
                *reinterpret_cast<uint32_t*>(&sB[buf][8 * c8 + 2 * b_ + 1][2 * rq]) = GM_BPAIR(h01); \
            }                                                                          \
        }                                                                              \
    } while (0)

    floatx4 acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    auto mma = [](half8 a, half8 b, floatx4 c) {
        if constexpr (XBF16)
            return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                           c, 0, 0, 0);
        else
            return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    };

    // Software pipeline over k steps, two LDS stages.  Entering iteration kt
    // a wave holds step kt's fragments in registers, LDS stage (kt+1)&1 holds
    // step kt+1 and the staging registers hold step kt+2's global data.
    // Iteration kt runs step kt's MFMAs with step kt+1's fragment reads
    // between them, stores step kt+2 into stage kt&1 (whose fragments every
    // wave read before the previous barrier) and issues step kt+3's global
    // loads; a barrier ends it.  The body is one basic block (the last
    // iterations load a clamped step and store it into a stage nobody reads
    // again), so the dequantization and the stores are scheduled between
    // the MFMAs.  The k-step order of each accumulator is unchanged.
    const int fr = lane & 15, fk = 8 * (lane >> 4);
    GM_GLOAD(0);
    GM_LSTORE(0);
    GM_GLOAD(min(1, nk - 1));
    GM_LSTORE(1);
    GM_GLOAD(min(2, nk - 1));
    __syncthreads();
    half8 af[MI], bfr[NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i) af[i] = *reinterpret_cast<const half8*>(&sA[0][16 * MI * wm + 16 * i + fr][fk]);
#pragma unroll
    for (int j = 0; j < NJ; ++j) bfr[j] = *reinterpret_cast<const half8*>(&sB[0][16 * NJ * wn + 16 * j + fr][fk]);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int nb = (kt + 1) & 1;
        half8 an[MI];
#pragma unroll
        for (int i = 0; i < MI; ++i) an[i] = *reinterpret_cast<const half8*>(&sA[nb][16 * MI * wm + 16 * i + fr][fk]);
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
#pragma unroll
            for (int i = 0; i < MI; ++i) acc[i][j] = mma(af[i], bfr[j], acc[i][j]);
            bfr[j] = *reinterpret_cast<const half8*>(&sB[nb][16 * NJ * wn + 16 * j + fr][fk]);
        }
        GM_LSTORE(kt & 1);
        GM_GLOAD(min(kt + 3, nk - 1));
        __builtin_amdgcn_iglp_opt(0);
#pragma unroll
        for (int i = 0; i < MI; ++i) af[i] = an[i];
        __syncthreads();
    }
#undef GM_GLOAD
#undef GM_LSTORE
#undef GM_BPAIR

    // Epilogue through LDS.  A C fragment gives a lane 4 rows of one column
    // (16 lanes: 32- or 64-byte pieces of a row), so each wave stages its
    // tile 16 rows at a time in a private region of the idle W stages (the
    // loop's last barrier ended every fragment read) and stores whole row
    // segments, 16 bytes of fp32 per lane.  A wave reads back only what it
    // wrote, and its LDS operations complete in order, so no barrier.  The
    // row stride OC + 4 keeps the 64 lanes' stores in distinct banks.
    constexpr int OC = GU ? 8 * NJ : 16 * NJ;              // output columns per wave
    constexpr int EPS = OC + 4;
    constexpr int LPR = OC / 4, RPI = 64 / LPR;            // lanes per staged row, rows per read
    static_assert(WM * WN * 16 * EPS * 4 <= (int)sizeof(sB), "epilogue staging");
    float* ep = reinterpret_cast<float*>(&sB[0][0][0]) + w * 16 * EPS;
    const int oc0 = n0 + OC * wn;
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
        for (int j = 0; j < NJ; j += (GU ? 2 : 1))
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // gate/up: fragments j, j + 1 are the gate and up values of the same outputs
                const float v = GU ? silu_fast(acc[i][j][e]) * acc[i][j + 1][e] : acc[i][j][e];
                ep[(4 * (lane >> 4) + e) * EPS + (GU ? 8 : 16) * j + fr] = v;
            }
#pragma unroll
        for (int r0 = 0; r0 < 16; r0 += RPI) {
            const int r = r0 + lane / LPR, c = 4 * (lane % LPR);
            const float4 v = *reinterpret_cast<const float4*>(&ep[r * EPS + c]);
            const int row = m0 + 16 * MI * wm + 16 * i + r, col = oc0 + c;
            if (row >= A.m || col >= A.n) continue;         // n % 32 == 0: the 4 columns are all in or all out
            const size_t o = (size_t)row * A.n + col;
            float4 y = v;
            if (!GU && A.residual) {
                const float4 rv = *reinterpret_cast<const float4*>(A.residual + o);
                y = make_float4(v.x + rv.x, v.y + rv.y, v.z + rv.z, v.w + rv.w);
            }
            if (GU || A.y_bf16)
                *reinterpret_cast<uint2*>(A.y_bf16 + o) =
                    make_uint2(pack_bf16x2(y.x, y.y), pack_bf16x2(y.z, y.w));
            else
                *reinterpret_cast<float4*>(A.y + o) = y;
        }
    }
}

extern "C" __global__ __launch_bounds__(256, 2) void qm_q4_gemm(Q4GemmArgs A) { q4_gemm_body<false, false, 2, 2, 4, 8>(A); }
extern "C" __global__ __launch_bounds__(256, 2) void qm_q4_gemm_xbf16(Q4GemmArgs A) { q4_gemm_body<true, false, 2, 2, 4, 8>(A); }
extern "C" __global__ __launch_bounds__(256, 2) void qm_q4_gemm_gu(Q4GemmArgs A) { q4_gemm_body<false, true, 2, 2, 4, 8>(A); }
extern "C" __global__ __launch_bounds__(256, 2) void qm_q4_gemm_gu_xbf16(Q4GemmArgs A) { q4_gemm_body<true, true, 2, 2, 4, 8>(A); }
extern "C" __global__ __launch_bounds__(256, 2) void qm_q4_gemm_n128(Q4GemmArgs A) { q4_gemm_body<false, false, 2, 2, 4, 4>(A); }
extern "C" __global__ __launch_bounds__(256, 2) void qm_q4_gemm_xbf16_n128(Q4GemmArgs A) { q4_gemm_body<true, false, 2, 2, 4, 4>(A); }
extern "C" __global__ __launch_bounds__(256, 2) void qm_q4_gemm_m64(Q4GemmArgs A) { q4_gemm_body<false, false, 2, 2, 2, 4>(A); }
extern "C" __global__ __launch_bounds__(256, 2) void qm_q4_gemm_xbf16_m64(Q4GemmArgs A) { q4_gemm_body<true, false, 2, 2, 2, 4>(A); }

// n = 32 (the DeltaNet a/b projections, 8-column device tiles): 4096 x 2560
// x 32 is too thin for LDS tiles, where each workgroup walks all k steps
// behind one chain of loads.  Here a workgroup of four waves owns 16 rows
// and deals the k steps to its waves round-robin.  Each wave builds its
// MFMA operands straight from global memory: the x row piece (lane: row
// lane & 15, k 8 (lane >> 4) .. +7) is the A operand as loaded; for the B
// operand of column c the lane loads rows k .. k+7 of c's tile (32
// contiguous bytes), takes nibble c & 7 of each and forms the f16 pairs
// s * (q - 8) with the same magic-number arithmetic as the staged form (for
// bf16 x, rounded on to bf16).  No LDS until the end, where the four
// partial sums meet and are added in a fixed order.
template <bool XBF16>
__device__ __forceinline__ void q4_gemm_n32_body(const Q4GemmArgs& A) {
    __shared__ floatx4 part[4][2][64];                   // [wave][column tile][lane]
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int m0 = (int)blockIdx.x * 16, K = A.k, nk = K / GM_TK;
    const int fr = lane & 15, kg = lane >> 4;
    const uint16_t* xr = A.x + (size_t)min(m0 + fr, A.m - 1) * K + 8 * kg;
    const int sh = 4 * (fr & 7);                         // nibble of column 16 j + fr in its row word
    const uint8_t* cb[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) cb[j] = A.codes + (size_t)(2 * j + (fr >> 3)) * K * 4 + 32 * kg;
    const uint16_t* sb = A.gscales + 8 * kg;             // one 32-column group: scales [k]
    uint32_t vmagic;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(vmagic));
    floatx4 acc[2] = {floatx4{0.0f, 0.0f, 0.0f, 0.0f}, floatx4{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll 4
    for (int kt = w; kt < nk; kt += 4) {
        const int k0 = kt * GM_TK;
        const half8 a = __builtin_bit_cast(half8, *reinterpret_cast<const uint4*>(xr + k0));
        const uint4 sc = *reinterpret_cast<const uint4*>(sb + k0);
        const uint32_t s4[4] = {sc.x, sc.y, sc.z, sc.w};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint4 c0 = *reinterpret_cast<const uint4*>(cb[j] + (size_t)k0 * 4);
            const uint4 c1 = *reinterpret_cast<const uint4*>(cb[j] + (size_t)k0 * 4 + 16);
            const uint32_t wd[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
            uint32_t bw[4];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint32_t q0 = (wd[2 * p] >> sh) & 0xfu, q1 = (wd[2 * p + 1] >> sh) & 0xfu;
                const half2 v = (__builtin_bit_cast(half2, (q0 | (q1 << 16)) | vmagic) - half2{1032.0f16, 1032.0f16}) *
                                __builtin_bit_cast(half2, s4[p]);
                bw[p] = XBF16 ? f16x2_to_bf16x2(v) : __builtin_bit_cast(uint32_t, v);
            }
            const half8 bv = __builtin_bit_cast(half8, make_uint4(bw[0], bw[1], bw[2], bw[3]));
            if constexpr (XBF16)
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, bv),
                                                                 acc[j], 0, 0, 0);
            else
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bv, acc[j], 0, 0, 0);
        }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) part[w][j][lane] = acc[j];
    __syncthreads();
    if (w != 0) return;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const floatx4 y = ((part[0][j][lane] + part[1][j][lane]) + part[2][j][lane]) + part[3][j][lane];
        const int col = 16 * j + fr;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int row = m0 + 4 * kg + e;
            if (row >= A.m) continue;
            const size_t o = (size_t)row * A.n + col;
            float v = y[e];
            if (A.residual) v += A.residual[o];
            if (A.y_bf16) A.y_bf16[o] = f32_to_bf16(v);
            else A.y[o] = v;
        }
    }
}
extern "C" __global__ __launch_bounds__(256) void qm_q4_gemm_n32(Q4GemmArgs A) { q4_gemm_n32_body<false>(A); }
extern "C" __global__ __launch_bounds__(256) void qm_q4_gemm_xbf16_n32(Q4GemmArgs A) { q4_gemm_n32_body<true>(A); }

// rms_norm (1 + gamma, eps 1e-6; gemv.rs:571-579) of each of m rows of f32
// x [m][k], written as the f16 input of qm_q4_gemm; without a norm weight,
// the plain f16 conversion.  One workgroup per row.
extern "C" __global__ __launch_bounds__(256) void qm_rms_norm_f16(RmsNormArgs A) {
    __shared__ float red[4];
    const int tid = threadIdx.x, row = blockIdx.x;
    const float* x = A.x + (size_t)row * A.k;
    float ss = 0.0f;
    for (int i = 4 * tid; i < A.k; i += 1024) {
        const float4 v = ld4(x + i);
        ss = fmaf(v.x, v.x, ss); ss = fmaf(v.y, v.y, ss); ss = fmaf(v.z, v.z, ss); ss = fmaf(v.w, v.w, ss);
    }
    ss = wave_sum64(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float inv = A.norm_w ? 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)A.k + 1e-6f) : 1.0f;
    uint16_t* out = A.out + (size_t)row * A.k;
    for (int i = 4 * tid; i < A.k; i += 1024) {
        const float4 v = ld4(x + i);
        float g[4] = {1.0f, 1.0f, 1.0f, 1.0f};
        if (A.norm_w) {
            const uint2 gw = *reinterpret_cast<const uint2*>(A.norm_w + i);
            g[0] = 1.0f + f16_to_f32((uint16_t)(gw.x & 0xffffu)); g[1] = 1.0f + f16_to_f32((uint16_t)(gw.x >> 16));
            g[2] = 1.0f + f16_to_f32((uint16_t)(gw.y & 0xffffu)); g[3] = 1.0f + f16_to_f32((uint16_t)(gw.y >> 16));
        }
        const uint32_t lo = (uint32_t)f32_to_f16(v.x * inv * g[0]) | ((uint32_t)f32_to_f16(v.y * inv * g[1]) << 16);
        const uint32_t hi = (uint32_t)f32_to_f16(v.z * inv * g[2]) | ((uint32_t)f32_to_f16(v.w * inv * g[3]) << 16);
        *reinterpret_cast<uint2*>(out + i) = make_uint2(lo, hi);
    }
}

