// qm_device.h -- gfx950 device helpers shared by the mixer kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define QM_DEV __device__ __forceinline__

// ---- cross-lane reductions (wave64; a DPP "row" is 16 lanes) -------------
// DPP controls: quad_perm[1,0,3,2] = 0xB1, quad_perm[2,3,0,1] = 0x4E,
// row_half_mirror = 0x141, row_mirror = 0x140.
template <int CTRL>
QM_DEV float dpp_f32(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Sum over the 16 lanes of a DPP row.  The result is bitwise identical in
// all 16 lanes (each step adds a commutative pair).
QM_DEV float row_sum16(float x) {
    x += dpp_f32<0xB1>(x);
    x += dpp_f32<0x4E>(x);
    x += dpp_f32<0x141>(x);
    x += dpp_f32<0x140>(x);
    return x;
}

QM_DEV float row_max16(float x) {
    x = fmaxf(x, dpp_f32<0xB1>(x));
    x = fmaxf(x, dpp_f32<0x4E>(x));
    x = fmaxf(x, dpp_f32<0x141>(x));
    x = fmaxf(x, dpp_f32<0x140>(x));
    return x;
}

QM_DEV float readlane_f32(float x, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}

// Sum over the whole wave: row sums then the four row results in a fixed
// order.  Uniform across the wave.
// Reductions with lane l ^ 16 / l ^ 32 through the gfx950 VALU row swaps
// (v_permlane16_swap / v_permlane32_swap): each lane ends up holding its own
// value and its partner's, in either order, so a commutative op of the pair
// is the reduction (no LDS round trip as with ds_bpermute).
QM_DEV float max_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
QM_DEV float max_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
QM_DEV float sum_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
QM_DEV float sum_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

QM_DEV float wave_sum64(float x) {
    x = row_sum16(x);
    float r0 = readlane_f32(x, 0), r1 = readlane_f32(x, 16);
    float r2 = readlane_f32(x, 32), r3 = readlane_f32(x, 48);
    return (r0 + r1) + (r2 + r3);
}

// ---- f16 / bf16 ----------------------------------------------------------
QM_DEV float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
QM_DEV uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
QM_DEV float bf16_to_f32(uint16_t h) { return __builtin_bit_cast(float, (uint32_t)h << 16); }
// f32 -> bf16, round to nearest even: one v_cvt_pk_bf16_f32 (gfx950) per
// pair of values, where the integer form (NaN test, bias, carry) took ~6
// VALU ops per value.  NaN stays NaN.
QM_DEV uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
QM_DEV uint32_t pack_bf16x2(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

// ---- scalar math (gemv.rs:631-659 semantics) -----------------------------
QM_DEV float silu_f(float x) { return x / (1.0f + expf(-x)); }

// The causal conv1d tap sum of gemv.rs:750-756 (and :1137-1142):
// ((b0 w0 + b1 w1) + b2 w2) + x w3 from zero, every product and sum rounded
// on its own as the reference's f32 arithmetic is.  The pragma is what keeps
// the compiler from contracting the pairs into FMAs (the __fmul_rn /
// __fadd_rn spellings do not).
QM_DEV float conv_taps4(float b0, float b1, float b2, float x, float4 w) {
#pragma clang fp contract(off)
    float s = 0.0f;
    s = s + b0 * w.x;
    s = s + b1 * w.y;
    s = s + b2 * w.z;
    s = s + x * w.w;
    return s;
}
// x * sigmoid(x) from v_exp_f32 (exp(-x) = 2^(-x log2 e)) and v_rcp_f32, a few
// ulp from silu_f; for the prefill paths, whose bar is bf16-level.
QM_DEV float silu_fast(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}
QM_DEV float softplus_f(float x) { return x > 20.0f ? x : logf(1.0f + expf(x)); }
// e^x and ln(1 + e^x) on v_exp_f32 / v_log_f32 (a few ulp from libm)
QM_DEV float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
QM_DEV float softplus_fast(float x) {
    return x > 20.0f ? x : __builtin_amdgcn_logf(1.0f + exp_fast(x)) * 0.6931471805599453f;
}
QM_DEV float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }
// 1 / (1 + 2^(-x log2 e)) on v_exp_f32 / v_rcp_f32 (about 1 ulp each)
QM_DEV float sigmoid_fast(float x) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}

// ---- memory helpers ------------------------------------------------------
QM_DEV float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
QM_DEV void st4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }

// 16 bytes per lane from global memory straight into LDS (LDS DMA): lane l
// writes lds + 16 l.  Issued as inline asm so that no compiler-inserted wait
// ties later LDS reads to it; the caller awaits completion explicitly
// (vmcnt) before the barrier that publishes the data.  It sets M0, so a
// kernel using it must have no other M0 user.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
QM_DEV void dma16(const void* gsrc, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(gsrc), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop
