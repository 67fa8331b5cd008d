// Translation unit of the VALU kernels (gather-dot, substrate fill) and their launchers.
#include "k44_launch.hpp"

namespace k44dev {

__global__ __launch_bounds__(256) void k44_fill_uniform_kernel(__half *dst, uint64_t rows,
                                                               uint32_t stride, uint32_t valid,
                                                               uint64_t pos0, uint64_t seed_mix) {
    const uint64_t total = rows * stride;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t r = i / stride;
        const uint32_t t = (uint32_t)(i - r * stride);
        float v = 0.0f;
        if (t < valid) {
            const uint64_t h = splitmix64((((pos0 + r) << 20) | t) ^ seed_mix);
            v = (float)((int32_t)(h >> 40) - 8388608) * (1.0f / 8388608.0f);
        }
        dst[i] = __float2half_rn(v);
    }
}


hipError_t launch_gather_dot(const GatherDotArgs &a, uint32_t slab, uint32_t ksplit,
                             uint32_t tokens, hipStream_t stream) {
    const dim3 grid(ksplit == 4u ? a.cout : (a.cout + 3u) / 4u, tokens / slab, 1u);
    const dim3 block(256u, 1u, 1u);
#define K44_GD(SLAB, U)                                                                        \
    if (ksplit == 4u)                                                                          \
        hipLaunchKernelGGL((k44_gather_dot_kernel<SLAB, U, 4>), grid, block, 0, stream, a);     \
    else                                                                                       \
        hipLaunchKernelGGL((k44_gather_dot_kernel<SLAB, U, 1>), grid, block, 0, stream, a);
    switch (slab) {
    case 256u: K44_GD(256, 16) break;
    case 128u: K44_GD(128, 8) break;
    case 64u: K44_GD(64, 4) break;
    default: return hipErrorInvalidValue;
    }
#undef K44_GD
    return hipGetLastError();
}

hipError_t launch_fill_uniform(__half *dst, uint64_t rows, uint32_t stride, uint32_t valid,
                               uint64_t pos0, uint64_t seed, hipStream_t stream) {
    const uint64_t total = rows * stride;
    const uint32_t blocks = (uint32_t)((total + 255u) / 256u < 65536u ? (total + 255u) / 256u : 65536u);
    hipLaunchKernelGGL(k44_fill_uniform_kernel, dim3(blocks ? blocks : 1u), dim3(256), 0, stream,
                       dst, rows, stride, valid, pos0, splitmix64(seed));
    return hipGetLastError();
}

}  // namespace k44dev
