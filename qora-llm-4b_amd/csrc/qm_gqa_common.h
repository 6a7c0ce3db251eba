// qm_gqa_common.h -- device helpers shared by the GQA decode and prefill kernels.
#pragma once
#include "qm_device.h"
#include "qm_kernel_args.h"

// Per-head RMSNorm (1+gamma, eps 1e-6; gemv.rs:586-597) and split-half RoPE
// (gemv.rs:604-627) of one 256-wide head held by a wave: lane owns dims
// 4*lane..4*lane+3.  Lanes 0..7 hold dims 0..31, lanes 8..15 dims 32..63,
// so rotation partners are 8 lanes apart inside DPP row 0 (row_ror:8).
// The inputs are loaded by the caller (rope_row_loads, the gamma row), so
// every load of a preparation can be issued before any of its arithmetic.
QM_DEV float4 norm_rope_head(float4 x, uint2 gw, float4 c, float4 s, int lane) {
    float ss = x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
    ss = wave_sum64(ss);
    const float inv = 1.0f / sqrtf(ss / (float)QM_GQA_HD + 1e-6f);
    x.x = x.x * inv * (1.0f + f16_to_f32((uint16_t)(gw.x & 0xffffu)));
    x.y = x.y * inv * (1.0f + f16_to_f32((uint16_t)(gw.x >> 16)));
    x.z = x.z * inv * (1.0f + f16_to_f32((uint16_t)(gw.y & 0xffffu)));
    x.w = x.w * inv * (1.0f + f16_to_f32((uint16_t)(gw.y >> 16)));
    float4 pr;
    pr.x = dpp_f32<0x128>(x.x);
    pr.y = dpp_f32<0x128>(x.y);
    pr.z = dpp_f32<0x128>(x.z);
    pr.w = dpp_f32<0x128>(x.w);
    // x1 c - x2 s (lanes 0..7, x1 own), x2 c + x1 s (lanes 8..15, x2 own)
    const float4 ps = lane < 8 ? make_float4(-pr.x, -pr.y, -pr.z, -pr.w) : pr;
    float4 y;
    y.x = x.x * c.x + ps.x * s.x;
    y.y = x.y * c.y + ps.y * s.y;
    y.z = x.z * c.z + ps.z * s.z;
    y.w = x.w * c.w + ps.w * s.w;
    return lane < 16 ? y : x;
}

// The cos / sin of lane's rotation index (every lane loads; lanes 0..15 use them).
QM_DEV void rope_row_loads(const float* cos_row, const float* sin_row, int lane, float4& c, float4& s) {
    const int i0 = (lane & 7) * 4;
    c = ld4(cos_row + i0);
    s = ld4(sin_row + i0);
}

