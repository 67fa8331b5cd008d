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


template <bool NTX>
static hipError_t launch_gather_dot_policy(const GatherDotArgs &a, uint32_t slab, uint32_t ksplit,
                                           uint32_t tokens, hipStream_t stream, bool lane8,
                                           bool weights_in_lds, bool misaligned) {
    const dim3 grid(ksplit == 4u ? a.cout : (a.cout + 3u) / 4u, tokens / slab, 1u);
    const dim3 block(256u, 1u, 1u);
    if (lane8 && misaligned) return hipErrorInvalidValue;  // 16-byte loads need aligned rows
    if (lane8) {
        const bool wl = weights_in_lds && (uint64_t)a.K * a.n_batch * 16u <= GD_WL_MAX;
#define K44_GD8(SLAB)                                                                                \
    if (ksplit == 4u) {                                                                              \
        if (wl) hipLaunchKernelGGL((k44_gather_dot8_kernel<SLAB, 4, NTX, true>), grid, block, 0, stream, a);  \
        else hipLaunchKernelGGL((k44_gather_dot8_kernel<SLAB, 4, NTX, false>), grid, block, 0, stream, a);    \
    } else {                                                                                         \
        if (wl) hipLaunchKernelGGL((k44_gather_dot8_kernel<SLAB, 1, NTX, true>), grid, block, 0, stream, a);  \
        else hipLaunchKernelGGL((k44_gather_dot8_kernel<SLAB, 1, NTX, false>), grid, block, 0, stream, a);    \
    }
        switch (slab) {
        case 256u: K44_GD8(256) break;
        case 128u: K44_GD8(128) break;
        case 64u: K44_GD8(64) break;
        default: return hipErrorInvalidValue;
        }
#undef K44_GD8
        return hipGetLastError();
    }
#define K44_GD(SLAB, U)                                                                          \
    if (misaligned) {                                                                            \
        if (ksplit == 4u)                                                                        \
            hipLaunchKernelGGL((k44_gather_dot_kernel<SLAB, U, 4, NTX, true>), grid, block, 0,    \
                               stream, a);                                                       \
        else                                                                                     \
            hipLaunchKernelGGL((k44_gather_dot_kernel<SLAB, U, 1, NTX, true>), grid, block, 0,    \
                               stream, a);                                                       \
    } else if (ksplit == 4u)                                                                     \
        hipLaunchKernelGGL((k44_gather_dot_kernel<SLAB, U, 4, NTX>), grid, block, 0, stream, a);  \
    else                                                                                         \
        hipLaunchKernelGGL((k44_gather_dot_kernel<SLAB, U, 1, NTX>), grid, block, 0, stream, a);
    switch (slab) {
    case 256u: K44_GD(256, 16) break;
    case 128u: K44_GD(128, 8) break;
    case 64u: K44_GD(64, 4) break;
    default: return hipErrorInvalidValue;
    }
#undef K44_GD
    return hipGetLastError();
}

hipError_t launch_gather_dot(const GatherDotArgs &a, uint32_t slab, uint32_t ksplit,
                             uint32_t tokens, hipStream_t stream, bool lane8, bool stream_loads,
                             bool weights_in_lds, bool misaligned) {
    return stream_loads ? launch_gather_dot_policy<true>(a, slab, ksplit, tokens, stream, lane8,
                                                         weights_in_lds, misaligned)
                        : launch_gather_dot_policy<false>(a, slab, ksplit, tokens, stream, lane8,
                                                          weights_in_lds, misaligned);
}

// Streaming gather kernel: 256 neurons x one 256-token slab per workgroup (16 waves, 128 KiB of
// LDS for the staged output rows).
hipError_t launch_gather_stream(const GatherDotArgs &a, uint32_t tokens, hipStream_t stream,
                                bool stream_loads) {
    // Measured on config 2 against 128 neurons x 16 / 8 waves and 256 x 8 waves: 2-5 % faster.
    constexpr uint32_t NPW = 256u, WAVES = 16u;
    const dim3 grid((a.cout + NPW - 1u) / NPW, tokens / 256u, 1u), block(WAVES * 64u, 1u, 1u);
    if (stream_loads)
        hipLaunchKernelGGL((k44_gather_stream_kernel<NPW, WAVES, true>), grid, block, 0, stream, a);
    else
        hipLaunchKernelGGL((k44_gather_stream_kernel<NPW, WAVES, false>), grid, block, 0, stream, a);
    return hipGetLastError();
}

// Split-K reduction + epilogue: workgroup (x, w) covers threads x*256.. of wave w of the group
// (grid.y = the group's waves, grid.x = the largest wave's workgroups: the wave is known without
// a table lookup); thread = (neuron j, 4 tokens); partials summed in z order.  Waves without
// split-K have no epilogue.  Every access goes through the global address space (pointers read
// from the descriptor would otherwise compile to flat accesses), and the cout_map entry, bias
// and the first 8 partial planes are loaded together, unconditionally (the partial buffer stands
// in for a null table; planes past the split re-read plane 0, unused), kept as raw bits until all
// are in flight: a load under a branch makes the compiler wait for it before the next.
__global__ __launch_bounds__(256) void k44_splitk_epilogue_kernel(K44_GROUP_PARAMS) {
    K44_GROUP_BIND;
    typedef const __attribute__((address_space(1))) f4_t gf4;
    typedef const __attribute__((address_space(1))) uint16_t gu16;
    typedef const __attribute__((address_space(1))) gd_u2 gu2;
    typedef __attribute__((address_space(1))) gd_u2 gu2w;
    const MfmaTileArgs a = grp.waves[blockIdx.y];
    // Every descriptor field the kernel reads is loaded before its first branch: a scalar load
    // placed after a uniform branch is issued only once the branch resolves, one round trip
    // to the descriptor per branch.
    asm volatile("" ::"s"(a.kgroups), "s"(a.arrive), "s"(a.cout), "s"(a.tokens), "s"(a.part), "s"(a.cmap),
                 "s"(a.bias), "s"(a.R), "s"(a.Y), "s"(a.out_stride), "s"(a.act), "s"(a.tile_y));
    const uint32_t groups = a.kgroups, cout = a.cout, tokens = a.tokens;
    if (groups <= 1u || a.arrive) return;  // unsplit, or reduced in its own launch
    const uint32_t per_row = tokens / 4u;
    const uint64_t q = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    const uint64_t nq = (uint64_t)cout * per_row;
    if (q >= nq) return;
    uint32_t j, t;
    if (nq <= 0xffffffffull) {  // 32-bit division (uniform)
        j = (uint32_t)q / per_row;
        t = ((uint32_t)q - j * per_row) * 4u;
    } else {
        j = (uint32_t)(q / per_row);
        t = (uint32_t)(q - (uint64_t)j * per_row) * 4u;
    }
    const uint64_t plane4 = (uint64_t)cout * tokens / 4u;
    gf4 *p = (gf4 *)(a.part + (uint64_t)j * tokens + t);
    gu16 *cm = (gu16 *)(a.cmap ? (const void *)a.cmap : (const void *)a.part);
    gu16 *bs = (gu16 *)(a.bias ? (const void *)a.bias : (const void *)a.part);
    uint32_t cbits = cm[j], bbits = bs[j];
    constexpr uint32_t U = 8u;
    f4_t u8[U];
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) u8[u] = p[(uint64_t)(u < groups ? u : 0u) * plane4];
    asm volatile("" : "+v"(cbits), "+v"(bbits));
    f4_t v = u8[0];
    const uint32_t first = groups < U ? groups : U;
    for (uint32_t u = 1; u < first; ++u) {  // z order
        v[0] += u8[u][0];
        v[1] += u8[u][1];
        v[2] += u8[u][2];
        v[3] += u8[u][3];
    }
    for (uint32_t z = U; z < groups; ++z) {
        const f4_t u1 = p[(uint64_t)z * plane4];
        v[0] += u1[0];
        v[1] += u1[1];
        v[2] += u1[2];
        v[3] += u1[3];
    }
    const uint64_t oj = a.cmap ? (uint64_t)cbits : (uint64_t)j;
    const float b = a.bias ? __half2float(__ushort_as_half((unsigned short)bbits)) : 0.0f;
    if (a.cmap && oj == K44_CMAP_EMPTY) return;
    const uint64_t o = oj * a.out_stride + tok_y(a, t);  // 4 tokens never cross a 64-token tile
    float r[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (a.R) {
        const gd_u2 rv = *(gu2 *)(a.R + o);
        const __half *rh = reinterpret_cast<const __half *>(&rv);
#pragma unroll
        for (int k = 0; k < 4; ++k) r[k] = __half2float(rh[k]);
    }
    const float acc[4] = {v[0], v[1], v[2], v[3]};
    __half out[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float s = acc[k] + b;
        out[k] = __float2half_rn(a.cmap ? apply_act(s + r[k], a.act) : apply_act(s, a.act) + r[k]);
    }
    *(gu2w *)(a.Y + o) = *reinterpret_cast<const gd_u2 *>(out);
}

hipError_t launch_splitk_epilogue(const MfmaGroup &g, uint32_t epi_max, hipStream_t stream) {
    if (epi_max == 0u) return hipSuccess;
    hipLaunchKernelGGL(k44_splitk_epilogue_kernel, dim3(epi_max, g.n), dim3(256), 0, stream, K44_GROUP_ARGS(g));
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
