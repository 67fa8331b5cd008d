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


hipError_t launch_gather_dot(const GatherDotArgs &a, uint32_t slab, uint32_t tokens,
                             hipStream_t stream) {
    const dim3 grid((a.cout + 3u) / 4u, tokens / slab, 1u), block(256u, 1u, 1u);
    switch (slab) {
    case 256u: hipLaunchKernelGGL((k44_gather_dot_kernel<256, 16>), grid, block, 0, stream, a); break;
    case 128u: hipLaunchKernelGGL((k44_gather_dot_kernel<128, 8>), grid, block, 0, stream, a); break;
    case 64u: hipLaunchKernelGGL((k44_gather_dot_kernel<64, 4>), grid, block, 0, stream, a); break;
    default: return hipErrorInvalidValue;
    }
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
