// Translation unit of the 2-D (spatial) kernels; semantics in k44_spatial.hpp.
#include "k44_gather_dot.hpp"
#include "k44_spatial.hpp"

namespace k44dev {

// 4 consecutive fp16 from an element offset of any alignment: two aligned 8-byte loads and a
// funnel shift (the 3x3 taps of a 2-D wave are shifted by +-1 element).  The second load may
// touch up to 3 elements past the last one used; the canvas carries slack for it.
__device__ __forceinline__ uint64_t load4_any(const __half *base, uint64_t e) {
    const uint32_t mis = (uint32_t)(e & 3u);
    const uint64_t *p = reinterpret_cast<const uint64_t *>(base + (e - mis));
    const uint64_t lo = p[0];
    if (mis == 0u) return lo;
    const uint64_t hi = p[1];
    return (lo >> (16u * mis)) | (hi << (64u - 16u * mis));
}

__device__ __forceinline__ void fma4_u64(float (&acc)[4], float w, uint64_t v) {
    const uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
    const float2 a = __half22float2(*reinterpret_cast<const __half2 *>(&lo));
    const float2 b = __half22float2(*reinterpret_cast<const __half2 *>(&hi));
    acc[0] = fmaf(w, a.x, acc[0]);
    acc[1] = fmaf(w, a.y, acc[1]);
    acc[2] = fmaf(w, b.x, acc[2]);
    acc[3] = fmaf(w, b.y, acc[3]);
}

// One wave = one neuron x one 64-token tile: lane (g, c) gathers tokens 4c..4c+3 of synapses
// g, g+4, ... (4 loads in flight), the 4 row groups meet via shuffles, 16 lanes store pixels.
__global__ __launch_bounds__(256) void k44_gather_tile_kernel(GatherTileArgs a) {
    const int lane = (int)(threadIdx.x & 63u), wave = (int)(threadIdx.x >> 6);
    const uint32_t j = blockIdx.x * 4u + (uint32_t)wave;
    if (j >= a.cout) return;
    const uint32_t c = (uint32_t)(lane & 15), g = (uint32_t)(lane >> 4);
    const uint64_t *seg = a.seg + (uint64_t)(j / a.cluster) * a.K;
    const uint32_t P = a.K * a.S;
    const __half *wj = a.W + (uint64_t)j * P;
    const float b = a.bias ? __half2float(a.bias[j]) : 0.0f;
    const uint64_t oj = a.cmap ? (uint64_t)a.cmap[j] : (uint64_t)j;
    for (uint32_t t = blockIdx.y; t < a.tiles; t += gridDim.y) {
        const uint64_t tx = a.tile_x[t] + 4u * c;
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (uint32_t p0 = g; p0 < P; p0 += 16u) {
            uint64_t v[4];
            float w[4];
            // every lane loads (positions past the row read its last position, replaced by zero
            // after the load): a load under the divergent branch would be waited for alone
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t p = p0 + 4u * (uint32_t)u;
                const uint32_t pc = p < P ? p : P - 1u;
                const uint32_t k = pc / a.S, s = pc - k * a.S;
                const uint64_t vl = load4_any(a.X, seg[k] + (uint64_t)s * a.step + tx);
                const float wl = __half2float(wj[pc]);
                v[u] = p < P ? vl : 0u;
                w[u] = p < P ? wl : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) fma4_u64(acc, w[u], v[u]);
        }
#pragma unroll
        for (int off = 16; off < 64; off <<= 1)
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[q] += __shfl_xor(acc[q], off, 64);
        if (g != 0u || (a.cmap && oj == K44_CMAP_EMPTY)) continue;
        const uint32_t tl = t % a.tiles_per_frame;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t m = 4u * c + (uint32_t)q;
            if (a.masked) {  // tile spans rows and halo columns: store pixels only
                const uint32_t rel = 64u * tl + m, row = rel / a.plane.W_pad;
                if (row >= a.plane.H || rel - row * a.plane.W_pad >= a.plane.W) continue;
            }
            const uint64_t o = oj * a.out_stride + a.tile_y[t] + m;
            const float r = a.R ? __half2float(a.R[o]) : 0.0f;
            const float v = acc[q] + b;
            a.Y[o] = __float2half_rn(a.cmap ? apply_act(v + r, a.act) : apply_act(v, a.act) + r);
        }
    }
}

__device__ __forceinline__ uint64_t pix(const Plane2D &p, uint32_t c, uint32_t f, uint32_t y,
                                        uint32_t x) {
    if (p.tok64)
        return (uint64_t)c * p.channel_stride + (uint64_t)(f >> 6) * 64u * p.single_stride +
               ((uint64_t)(y + 1u) * p.W_pad + x + 1u) * 64u + (f & 63u);
    return (uint64_t)c * p.channel_stride + (uint64_t)f * p.single_stride +
           (uint64_t)(y + 1u) * p.W_pad + 4u + x;
}

// Grid-stride over (channel, frame, y, x) of an H x W x frames x C index space.
#define K44_FOR_PIXELS(C, P)                                                                     \
    const uint64_t n_ = (uint64_t)(C) * (P).frames * (P).H * (P).W;                               \
    for (uint64_t i_ = (uint64_t)blockIdx.x * 256u + threadIdx.x; i_ < n_;                        \
         i_ += (uint64_t)gridDim.x * 256u)

#define K44_SPLIT_PIXEL(P)                                                                       \
    const uint32_t x = (uint32_t)(i_ % (P).W);                                                    \
    const uint64_t r1_ = i_ / (P).W;                                                              \
    const uint32_t y = (uint32_t)(r1_ % (P).H);                                                   \
    const uint64_t r2_ = r1_ / (P).H;                                                             \
    const uint32_t f = (uint32_t)(r2_ % (P).frames);                                              \
    const uint32_t c = (uint32_t)(r2_ / (P).frames);

// Planes: (channel, frame) of single_stride elements, or (channel, 64-frame block) of
// 64 * single_stride elements in the interleaved layout (element e belongs to pixel e / 64).
__global__ __launch_bounds__(256) void k44_halo_clear_kernel(__half *base, uint32_t planes,
                                                             Plane2D p) {
    const uint32_t per_ch = p.tok64 ? p.frames / 64u : p.frames;
    const uint64_t plane = p.tok64 ? 64u * p.single_stride : p.single_stride;
    const uint32_t sh = p.tok64 ? 6u : 0u, col0 = p.tok64 ? 1u : 4u;
    for (uint32_t pl = blockIdx.y; pl < planes; pl += gridDim.y) {
        const uint32_t c = pl / per_ch, f = pl - c * per_ch;
        __half *pb = base + (uint64_t)c * p.channel_stride + (uint64_t)f * plane;
        for (uint64_t e = (uint64_t)blockIdx.x * 256u + threadIdx.x; e < plane;
             e += (uint64_t)gridDim.x * 256u) {
            const uint64_t px = e >> sh, row = px / p.W_pad, col = px - row * p.W_pad;
            if (row >= 1u && row <= p.H && col >= col0 && col < col0 + p.W) continue;
            pb[e] = __float2half_rn(0.0f);
        }
    }
}

__global__ __launch_bounds__(256) void k44_s2d_kernel(__half *yo, const __half *xi, uint32_t cin,
                                                      Plane2D in, Plane2D out) {
    K44_FOR_PIXELS(cin, out) {
        K44_SPLIT_PIXEL(out)
#pragma unroll
        for (uint32_t py = 0; py < 2u; ++py)
#pragma unroll
            for (uint32_t px = 0; px < 2u; ++px) {  // zero padding past the input's edge
                const uint32_t yy = 2u * y + py, xx = 2u * x + px;
                yo[pix(out, 4u * c + 2u * py + px, f, y, x)] =
                    (yy < in.H && xx < in.W) ? xi[pix(in, c, f, yy, xx)] : __float2half_rn(0.0f);
            }
    }
}

__global__ __launch_bounds__(256) void k44_maxpool2_kernel(__half *yo, const __half *xi,
                                                           uint32_t ch, Plane2D in, Plane2D out) {
    K44_FOR_PIXELS(ch, out) {
        K44_SPLIT_PIXEL(out)
        const float a = __half2float(xi[pix(in, c, f, 2u * y, 2u * x)]);
        const float b = __half2float(xi[pix(in, c, f, 2u * y, 2u * x + 1u)]);
        const float d = __half2float(xi[pix(in, c, f, 2u * y + 1u, 2u * x)]);
        const float e = __half2float(xi[pix(in, c, f, 2u * y + 1u, 2u * x + 1u)]);
        yo[pix(out, c, f, y, x)] = __float2half_rn(fmaxf(fmaxf(a, b), fmaxf(d, e)));
    }
}

__global__ __launch_bounds__(256) void k44_maxpool5_kernel(__half *yo, const __half *xi,
                                                           uint32_t ch, Plane2D in, Plane2D out) {
    K44_FOR_PIXELS(ch, out) {
        K44_SPLIT_PIXEL(out)
        float m = -INFINITY;
        for (int dy = -2; dy <= 2; ++dy) {
            const int yy = (int)y + dy;
            if (yy < 0 || yy >= (int)in.H) continue;
            for (int dx = -2; dx <= 2; ++dx) {
                const int xx = (int)x + dx;
                if (xx < 0 || xx >= (int)in.W) continue;
                m = fmaxf(m, __half2float(xi[pix(in, c, f, (uint32_t)yy, (uint32_t)xx)]));
            }
        }
        yo[pix(out, c, f, y, x)] = __float2half_rn(m);
    }
}

__global__ __launch_bounds__(256) void k44_upsample2_kernel(__half *yo, const __half *xi,
                                                            uint32_t ch, Plane2D in, Plane2D out) {
    K44_FOR_PIXELS(ch, out) {
        K44_SPLIT_PIXEL(out)
        yo[pix(out, c, f, y, x)] = xi[pix(in, c, f, y / 2u, x / 2u)];
    }
}

__global__ __launch_bounds__(256) void k44_scatter_up2_kernel(__half *yo, const __half *xi,
                                                              uint32_t cout, uint32_t qstride,
                                                              Plane2D in, Plane2D out) {
    K44_FOR_PIXELS(cout, out) {
        K44_SPLIT_PIXEL(out)
        const uint32_t q = 2u * (y & 1u) + (x & 1u);
        yo[pix(out, c, f, y, x)] = xi[pix(in, q * qstride + c, f, y / 2u, x / 2u)];
    }
}

static dim3 grid_pixels(uint64_t n) {
    const uint64_t b = (n + 255u) / 256u;
    return dim3((uint32_t)(b == 0 ? 1 : (b < 65536u ? b : 65536u)));
}

hipError_t launch_gather_tile(const GatherTileArgs &a, hipStream_t stream) {
    if (a.tiles == 0u || a.cout == 0u) return hipSuccess;
    const dim3 grid((a.cout + 3u) / 4u, a.tiles < 65535u ? a.tiles : 65535u);
    hipLaunchKernelGGL(k44_gather_tile_kernel, grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_halo_clear(__half *base, uint32_t channels, const Plane2D &p,
                             hipStream_t stream) {
    if (p.tok64 && p.frames % 64u != 0u) return hipErrorInvalidValue;
    const uint32_t planes = channels * (p.tok64 ? p.frames / 64u : p.frames);
    if (planes == 0u) return hipSuccess;
    const uint64_t bx = ((p.tok64 ? 64u : 1u) * p.single_stride + 255u) / 256u;
    const dim3 grid((uint32_t)(bx < 4096u ? bx : 4096u), planes < 65535u ? planes : 65535u);
    hipLaunchKernelGGL(k44_halo_clear_kernel, grid, dim3(256), 0, stream, base, planes, p);
    return hipGetLastError();
}

hipError_t launch_s2d(__half *y, const __half *x, uint32_t cin, const Plane2D &in,
                      const Plane2D &out, hipStream_t stream) {
    hipLaunchKernelGGL(k44_s2d_kernel, grid_pixels((uint64_t)cin * out.frames * out.H * out.W),
                       dim3(256), 0, stream, y, x, cin, in, out);
    return hipGetLastError();
}

hipError_t launch_maxpool2(__half *y, const __half *x, uint32_t c, const Plane2D &in,
                           const Plane2D &out, hipStream_t stream) {
    hipLaunchKernelGGL(k44_maxpool2_kernel, grid_pixels((uint64_t)c * out.frames * out.H * out.W),
                       dim3(256), 0, stream, y, x, c, in, out);
    return hipGetLastError();
}

hipError_t launch_maxpool5(__half *y, const __half *x, uint32_t c, const Plane2D &in,
                           const Plane2D &out, hipStream_t stream) {
    hipLaunchKernelGGL(k44_maxpool5_kernel, grid_pixels((uint64_t)c * out.frames * out.H * out.W),
                       dim3(256), 0, stream, y, x, c, in, out);
    return hipGetLastError();
}

hipError_t launch_upsample2(__half *y, const __half *x, uint32_t c, const Plane2D &in,
                            const Plane2D &out, hipStream_t stream) {
    hipLaunchKernelGGL(k44_upsample2_kernel, grid_pixels((uint64_t)c * out.frames * out.H * out.W),
                       dim3(256), 0, stream, y, x, c, in, out);
    return hipGetLastError();
}

hipError_t launch_scatter_up2(__half *y, const __half *x, uint32_t cout, uint32_t qstride,
                              const Plane2D &in, const Plane2D &out, hipStream_t stream) {
    hipLaunchKernelGGL(k44_scatter_up2_kernel,
                       grid_pixels((uint64_t)cout * out.frames * out.H * out.W), dim3(256), 0,
                       stream, y, x, cout, qstride, in, out);
    return hipGetLastError();
}

}  // namespace k44dev
