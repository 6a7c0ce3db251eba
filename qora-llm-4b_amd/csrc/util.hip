// util.hip -- synthetic-data fill for benchmarks and device-side tests.
// Not a mixer op: a counter-based N(mean, std) generator so that multi-GB
// synthetic caches can be filled in HBM without a host round trip.
#include "qm_device.h"
#include "qm_kernel_args.h"

QM_DEV uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Element i gets Box-Muller of two 24-bit uniforms from splitmix64(seed, i).
extern "C" __global__ __launch_bounds__(256) void qm_fill_normal(FillArgs A) {
    const uint64_t stride = (uint64_t)gridDim.x * 256u;
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < A.count; i += stride) {
        const uint64_t r = splitmix64(A.seed * 0xD1B54A32D192ED03ull + i);
        const float u1 = ((float)(uint32_t)(r >> 40) + 0.5f) * (1.0f / 16777216.0f);
        const float u2 = (float)(uint32_t)((r >> 16) & 0xffffffu) * (1.0f / 16777216.0f);
        const float n = sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
        const float x = A.mean + A.stdev * n;
        if (A.dtype == 0) static_cast<float*>(A.dst)[i] = x;
        else if (A.dtype == 1) static_cast<uint16_t*>(A.dst)[i] = f32_to_f16(x);
        else static_cast<uint16_t*>(A.dst)[i] = f32_to_bf16(x);
    }
}
