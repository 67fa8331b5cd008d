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

// Split-K reduction + epilogue: thread = (neuron j, 4 tokens); partials summed in z order.
__global__ __launch_bounds__(256) void k44_splitk_epilogue_kernel(
    const float *__restrict__ part, uint32_t groups, uint32_t cout, uint32_t tokens,
    const __half *__restrict__ bias, const uint16_t *__restrict__ cmap, const __half *R,
    __half *Y, uint32_t out_stride, int act) {
    const uint32_t per_row = tokens / 4u;
    const uint64_t q = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (q >= (uint64_t)cout * per_row) return;
    const uint32_t j = (uint32_t)(q / per_row), t = (uint32_t)(q - (uint64_t)j * per_row) * 4u;
    const uint64_t oj = cmap ? (uint64_t)cmap[j] : (uint64_t)j;
    if (oj == K44_CMAP_EMPTY) return;
    const uint64_t plane4 = (uint64_t)cout * tokens / 4u;
    const float4 *p = reinterpret_cast<const float4 *>(part + (uint64_t)j * tokens + t);
    float4 v = p[0];
    uint32_t z = 1;
    for (; z + 8u <= groups; z += 8u) {  // 8 partial loads in flight, summed in z order
        float4 w[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) w[u] = p[(uint64_t)(z + u) * plane4];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            v.x += w[u].x;
            v.y += w[u].y;
            v.z += w[u].z;
            v.w += w[u].w;
        }
    }
    for (; z < groups; ++z) {
        const float4 w = p[(uint64_t)z * plane4];
        v.x += w.x;
        v.y += w.y;
        v.z += w.z;
        v.w += w.w;
    }
    const float b = bias ? __half2float(bias[j]) : 0.0f;
    const uint64_t o = oj * out_stride + t;
    float r[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (R) {
        const gd_u2 rv = *reinterpret_cast<const gd_u2 *>(R + o);
        const __half *rh = reinterpret_cast<const __half *>(&rv);
#pragma unroll
        for (int k = 0; k < 4; ++k) r[k] = __half2float(rh[k]);
    }
    const float acc[4] = {v.x, v.y, v.z, v.w};
    __half out[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float s = acc[k] + b;
        out[k] = __float2half_rn(cmap ? apply_act(s + r[k], act) : apply_act(s, act) + r[k]);
    }
    *reinterpret_cast<gd_u2 *>(Y + o) = *reinterpret_cast<const gd_u2 *>(out);
}

hipError_t launch_splitk_epilogue(const MfmaTileArgs &a, uint32_t groups, hipStream_t stream) {
    if (!a.part || a.tokens % 4u != 0u) return hipErrorInvalidValue;
    const uint64_t n = (uint64_t)a.cout * (a.tokens / 4u);
    hipLaunchKernelGGL(k44_splitk_epilogue_kernel, dim3((uint32_t)((n + 255u) / 256u)),
                       dim3(256), 0, stream, a.part, groups, a.cout, a.tokens, a.bias, a.cmap,
                       a.R, a.Y, a.out_stride, a.act);
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
