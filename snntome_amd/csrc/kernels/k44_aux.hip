// Translation unit of the 1-D token ops (see k44_aux.hpp for their semantics).
#include "k44_aux.hpp"

namespace k44dev {

// One workgroup per 64-token tile: 256 threads = 8 token-octets x 32 channel lanes.  Each thread
// reads 16-byte runs of 8 tokens down its channel stripe, sums squares per token, the 32 stripes
// of a token octet reduce through LDS, and the same threads write the normalised values.
__global__ __launch_bounds__(256) void k44_rmsnorm_kernel(__half *__restrict__ y,
                                                          const __half *__restrict__ x,
                                                          const __half *__restrict__ gamma,
                                                          uint32_t D, uint32_t stride, float eps) {
    __shared__ float part[32][65];
    const uint32_t oct = threadIdx.x & 7u, lane_c = threadIdx.x >> 3;
    const uint32_t t0 = blockIdx.x * 64u + oct * 8u;
    float ss[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (uint32_t c = lane_c; c < D; c += 32u) {
        const uint4 v = *reinterpret_cast<const uint4 *>(x + (uint64_t)c * stride + t0);
        const __half *h = reinterpret_cast<const __half *>(&v);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float f = __half2float(h[k]);
            ss[k] = fmaf(f, f, ss[k]);
        }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) part[lane_c][oct * 8u + k] = ss[k];
    __syncthreads();
    float inv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        float tot = 0.0f;
        for (int r = 0; r < 32; ++r) tot += part[r][oct * 8u + k];
        inv[k] = rsqrtf(tot / (float)D + eps);
    }
    for (uint32_t c = lane_c; c < D; c += 32u) {
        const uint4 v = *reinterpret_cast<const uint4 *>(x + (uint64_t)c * stride + t0);
        const __half *h = reinterpret_cast<const __half *>(&v);
        const float g = gamma ? __half2float(gamma[c]) : 1.0f;
        uint4 o;
        __half *oh = reinterpret_cast<__half *>(&o);
#pragma unroll
        for (int k = 0; k < 8; ++k) oh[k] = __float2half_rn(__half2float(h[k]) * inv[k] * g);
        *reinterpret_cast<uint4 *>(y + (uint64_t)c * stride + t0) = o;
    }
}

__global__ __launch_bounds__(256) void k44_mul_kernel(__half *__restrict__ y,
                                                      const __half *__restrict__ a,
                                                      const __half *__restrict__ b, uint64_t n8) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < n8;
         i += (uint64_t)gridDim.x * 256u) {
        const uint4 va = reinterpret_cast<const uint4 *>(a)[i];
        const uint4 vb = reinterpret_cast<const uint4 *>(b)[i];
        const __half *ha = reinterpret_cast<const __half *>(&va);
        const __half *hb = reinterpret_cast<const __half *>(&vb);
        uint4 o;
        __half *ho = reinterpret_cast<__half *>(&o);
#pragma unroll
        for (int k = 0; k < 8; ++k) ho[k] = __float2half_rn(__half2float(ha[k]) * __half2float(hb[k]));
        reinterpret_cast<uint4 *>(y)[i] = o;
    }
}

// One thread per (channel, token).  State block of channel c: state[(c*(rf-1) + i)*64 + r] =
// input of request r, i+1 tokens back.
__global__ __launch_bounds__(256) void k44_token_shift_kernel(
    __half *__restrict__ y, const __half *__restrict__ x, const __half *__restrict__ mu,
    __half *__restrict__ state, uint32_t D, uint32_t stride, uint32_t tokens, uint32_t rf,
    uint32_t seq_len, int decode) {
    const uint64_t n = (uint64_t)D * stride;
    for (uint64_t e = (uint64_t)blockIdx.x * 256u + threadIdx.x; e < n;
         e += (uint64_t)gridDim.x * 256u) {
        const uint32_t c = (uint32_t)(e / stride), t = (uint32_t)(e - (uint64_t)c * stride);
        const __half *m = mu + (uint64_t)c * rf;
        const float xt = __half2float(x[e]);
        float acc = __half2float(m[0]) * xt;
        if (t >= tokens) {
            y[e] = __float2half_rn(0.0f);
            continue;
        }
        if (decode) {
            __half *st = state + (uint64_t)c * (rf - 1u) * 64u + t;  // request r = token t
            float prev[8];
            for (uint32_t i = 1; i < rf; ++i) prev[i - 1] = __half2float(st[(i - 1u) * 64u]);
            for (uint32_t i = 1; i < rf; ++i) acc = fmaf(__half2float(m[i]), prev[i - 1], acc);
            for (uint32_t i = rf - 1u; i > 1u; --i) st[(i - 1u) * 64u] = __float2half_rn(prev[i - 2]);
            if (rf > 1u) st[0] = x[e];
        } else {
            const uint32_t pos = t % seq_len;
            for (uint32_t i = 1; i < rf && i <= pos; ++i)
                acc = fmaf(__half2float(m[i]), __half2float(x[e - i]), acc);
            if (state && pos + rf > seq_len) {  // last rf-1 tokens of the request -> state
                const uint32_t back = seq_len - 1u - pos;  // 0 = newest
                if (back < rf - 1u) {
                    const uint32_t r = t / seq_len;
                    state[((uint64_t)c * (rf - 1u) + back) * 64u + r] = x[e];
                }
            }
        }
        y[e] = __float2half_rn(acc);
    }
}

__global__ __launch_bounds__(256) void k44_embed_kernel(__half *__restrict__ y,
                                                        const __half *__restrict__ table,
                                                        const uint32_t *__restrict__ ids,
                                                        uint32_t D, uint32_t vocab,
                                                        uint32_t stride, uint32_t tokens) {
    const uint64_t n = (uint64_t)D * stride;
    for (uint64_t e = (uint64_t)blockIdx.x * 256u + threadIdx.x; e < n;
         e += (uint64_t)gridDim.x * 256u) {
        const uint32_t c = (uint32_t)(e / stride), t = (uint32_t)(e - (uint64_t)c * stride);
        __half v = __float2half_rn(0.0f);
        if (t < tokens) {
            const uint32_t id = ids[t];
            if (id < vocab) v = table[(uint64_t)id * D + c];
        }
        y[e] = v;
    }
}

// One workgroup per token: 256 threads scan the vocabulary with a stride, then reduce
// (value, index) pairs in LDS; ties resolve to the lowest index.
__global__ __launch_bounds__(256) void k44_argmax_kernel(uint32_t *__restrict__ ids,
                                                         uint32_t *__restrict__ history,
                                                         const uint32_t *__restrict__ step_ctr,
                                                         uint32_t hist_steps, uint32_t tokens,
                                                         const __half *__restrict__ x, uint32_t V,
                                                         uint32_t stride) {
    __shared__ float bv[256];
    __shared__ uint32_t bi[256];
    const uint32_t t = blockIdx.x;
    float best = -INFINITY;
    uint32_t arg = 0xffffffffu;
    for (uint32_t c = threadIdx.x; c < V; c += 256u) {
        const float v = __half2float(x[(uint64_t)c * stride + t]);
        if (v > best || (v == best && c < arg)) {
            best = v;
            arg = c;
        }
    }
    bv[threadIdx.x] = best;
    bi[threadIdx.x] = arg;
    __syncthreads();
    for (uint32_t s = 128u; s > 0u; s >>= 1) {
        if (threadIdx.x < s) {
            const float v = bv[threadIdx.x + s];
            const uint32_t i = bi[threadIdx.x + s];
            if (v > bv[threadIdx.x] || (v == bv[threadIdx.x] && i < bi[threadIdx.x])) {
                bv[threadIdx.x] = v;
                bi[threadIdx.x] = i;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const uint32_t id = bi[0] == 0xffffffffu ? 0u : bi[0];
        ids[t] = id;
        if (history) {
            const uint32_t step = *step_ctr;
            if (step < hist_steps) history[(uint64_t)step * tokens + t] = id;
        }
    }
}

static uint32_t grid_for(uint64_t n) {
    const uint64_t b = (n + 255u) / 256u;
    return (uint32_t)(b == 0 ? 1 : (b < 65536u ? b : 65536u));
}

hipError_t launch_rmsnorm(__half *y, const __half *x, const __half *gamma, uint32_t D,
                          uint32_t stride, uint32_t tokens, float eps, hipStream_t stream) {
    (void)tokens;
    if (stride % 64u != 0u) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k44_rmsnorm_kernel, dim3(stride / 64u), dim3(256), 0, stream, y, x, gamma,
                       D, stride, eps);
    return hipGetLastError();
}

hipError_t launch_mul(__half *y, const __half *a, const __half *b, uint64_t n,
                      hipStream_t stream) {
    if (n % 8u != 0u) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k44_mul_kernel, dim3(grid_for(n / 8u)), dim3(256), 0, stream, y, a, b,
                       n / 8u);
    return hipGetLastError();
}

hipError_t launch_token_shift(__half *y, const __half *x, const __half *mu, __half *state,
                              uint32_t D, uint32_t stride, uint32_t tokens, uint32_t rf,
                              uint32_t seq_len, int decode, hipStream_t stream) {
    if (rf == 0u || rf > 9u || seq_len == 0u || (decode && (!state || tokens > 64u)))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k44_token_shift_kernel, dim3(grid_for((uint64_t)D * stride)), dim3(256), 0,
                       stream, y, x, mu, state, D, stride, tokens, rf, seq_len, decode);
    return hipGetLastError();
}

hipError_t launch_embed(__half *y, const __half *table, const uint32_t *ids, uint32_t D,
                        uint32_t vocab, uint32_t stride, uint32_t tokens, hipStream_t stream) {
    hipLaunchKernelGGL(k44_embed_kernel, dim3(grid_for((uint64_t)D * stride)), dim3(256), 0,
                       stream, y, table, ids, D, vocab, stride, tokens);
    return hipGetLastError();
}

__global__ void k44_step_inc_kernel(uint32_t *ctr) { *ctr += 1u; }

hipError_t launch_argmax(uint32_t *ids, uint32_t *history, uint32_t *step_ctr,
                         uint32_t hist_steps, const __half *x, uint32_t V, uint32_t stride,
                         uint32_t tokens, hipStream_t stream) {
    hipLaunchKernelGGL(k44_argmax_kernel, dim3(tokens), dim3(256), 0, stream, ids, history,
                       step_ctr, hist_steps, tokens, x, V, stride);
    if (history) hipLaunchKernelGGL(k44_step_inc_kernel, dim3(1), dim3(1), 0, stream, step_ctr);
    return hipGetLastError();
}

}  // namespace k44dev
