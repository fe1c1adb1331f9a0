// Small kernels that only the host side launches (placement probe, input
// staging, synthetic data), compiled in leap_hip_attention.hip alone.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace leap {

// ---- placement probe ---------------------------------------------------------

// The XCC (XCD) each workgroup runs on, from the hardware register XCC_ID
// (bits 3:0): xcc[blockIdx.x].  The decode kernel's merge keeps a group's
// partials in one XCD's L2 on the assumption that workgroup ids equal modulo
// kXcds land on the same XCD; create checks that with this probe.
__global__ void xcc_probe_kernel(int *xcc)
{
    if (threadIdx.x == 0) {
        unsigned v;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
        xcc[blockIdx.x] = (int)(v & 0xFu);
    }
}

// ---- synthetic data ---------------------------------------------------------

__device__ __forceinline__ uint64_t splitmix64(uint64_t x)
{
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// Copy n16 16-byte words from device-accessible (pinned) host memory: the
// host-pointer entry points stage their few KB of inputs this way, reading
// across PCIe from the kernel instead of a DMA-engine copy.
__global__ void stage_in_kernel(float4 *__restrict__ dst, const float4 *__restrict__ src, int n16)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n16) dst[i] = src[i];
}

// Two N(0,1) values per counter (Box-Muller on two 24-bit uniforms).
__global__ void fill_normal_kernel(float *dst, size_t n, uint64_t seed, float scale)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x * 2;
    for (size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 2; i < n; i += stride) {
        const uint64_t r = splitmix64(seed ^ splitmix64(i));
        const float u1 = ((float)(r >> 40) + 1.0f) * (1.0f / 16777216.0f);  // (0, 1]
        const float u2 = (float)((r >> 16) & 0xFFFFFF) * (1.0f / 16777216.0f);
        const float rad = sqrtf(-2.0f * logf(u1)) * scale;
        float sn, cs;
        sincosf(6.28318530717958647692f * u2, &sn, &cs);
        dst[i] = rad * cs;
        if (i + 1 < n) dst[i + 1] = rad * sn;
    }
}

}  // namespace leap
