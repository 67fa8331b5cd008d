// k44_gather_dot.hpp — VALU gather-dot wave kernel for gfx950 (wave64).
//
// Computes one K44_WAVE command on a 1-D token canvas (semantics of the reference's
// kernels/rocm/kernel44_rocm_pack.cuh:145-237, re-designed for CDNA4):
//   v[j][m] = bias[j] + sum_k sum_s W[j][k*S+s] * X[seg[j/cluster][k] + s*step + m]
//   y       = cmap ? act(v + r) : act(v) + r        (r = residual, 0 if none)
//   Y[y_off + out_j*out_stride + m] = fp16_rne(y),  out_j = cmap ? cmap[j] : j
//   (cmap[j] = 0xFFFF: empty slot, nothing stored)
// Used for waves whose neurons do not share index rows (per-neuron dendritic clusters): there
// is no dense contraction to hand to MFMA, the wave is a batched GEMV streaming 2*M bytes per
// gathered position, bound by HBM (or MALL/L2 when the substrate is cache resident).
//
// Mapping.  One wave64 = one neuron x one slab of SLAB tokens.  A position row of the slab is
// SLAB*2 contiguous bytes; lane = (g, c) with c = 4-token chunk (8 bytes) and g = row group, so
// one load instruction reads RPI = 256/SLAB rows of the segment, fully coalesced.  Rows are
// consumed in batches of RPI*U: every lane issues U independent 8-byte loads before the first
// FMA (U = 16/RPI loads in flight per lane), and one aligned vector load of the U weights it
// needs — the host stores W in exactly this batch order ([j][k][batch][g][u], zero padded), so
// weight traffic is one 8..32-byte load per lane per batch.  Row groups are reduced with
// cross-lane shuffles at the end; group 0 runs the fused epilogue and stores 8 bytes per lane.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace k44dev {

// Address-space-qualified views: read-only tables through the constant space (scalar loads),
// data through the global space (a generic pointer loaded from memory would compile to flat
// loads, which also count against the LDS wait counter).
typedef const __attribute__((address_space(1))) void kglobal_void;
typedef const __attribute__((address_space(4))) uint64_t kconst_u64;
typedef const __attribute__((address_space(4))) uint32_t kconst_u32;

// The aligned 32-bit word holding element j of a 16-bit table, by a scalar load issued
// unconditionally (`fallback`, any buffer of >= 2*(j+1) bytes, stands in for a null table), so
// that it completes under the gathers that follow instead of in a branch before them.  Tables
// are 4-byte aligned with an even element count (neuron counts are padded to multiples of 16).
__device__ __forceinline__ uint32_t scalar_word16(const void *table, const void *fallback,
                                                  uint32_t j) {
    return ((const kconst_u32 *)(table ? table : fallback))[j >> 1];
}
__device__ __forceinline__ uint32_t half_of(uint32_t word, uint32_t j) {
    return (j & 1u) ? (word >> 16) : (word & 0xffffu);
}

enum : int { ACT_NONE = 0, ACT_RELU = 1, ACT_SIGMOID = 2, ACT_SILU = 3, ACT_LEAKY = 4, ACT_GELU = 5 };

// cout_map entry of an empty slot (a pattern-sorted tile with fewer neurons than slots): the
// epilogue stores nothing for it.  Only with a cout_map: without one, neuron 65535 of a large
// wave is an ordinary output channel.
constexpr uint64_t K44_CMAP_EMPTY = 0xffffu;

// Largest per-neuron weight block (halves) the gather kernels stage in LDS.
constexpr uint32_t GD_WL_MAX = 2048;

// Activation with the id fixed at compile time (epilogues that apply it many times in
// unrolled code instantiate one activation instead of inlining the whole switch per element,
// which multiplies the code size past the instruction cache).
template <int ACT>
__device__ __forceinline__ float act_c(float v) {
    if constexpr (ACT == ACT_RELU) return fmaxf(v, 0.0f);
    else if constexpr (ACT == ACT_SIGMOID) return 1.0f / (1.0f + __expf(-v));
    else if constexpr (ACT == ACT_SILU) return v / (1.0f + __expf(-v));
    else if constexpr (ACT == ACT_LEAKY) return fmaxf(v, 0.1f * v);
    else if constexpr (ACT == ACT_GELU) return 0.5f * v * (1.0f + erff(v * 0.70710678f));
    else return v;
}

__device__ __forceinline__ float apply_act(float v, int act) {
    switch (act) {
    case ACT_RELU: return act_c<ACT_RELU>(v);
    case ACT_SIGMOID: return act_c<ACT_SIGMOID>(v);
    case ACT_SILU: return act_c<ACT_SILU>(v);
    case ACT_LEAKY: return act_c<ACT_LEAKY>(v);
    case ACT_GELU: return act_c<ACT_GELU>(v);
    default: return act_c<ACT_NONE>(v);
    }
}

// Runs the statement(s) with the activation id of `act` as the compile-time constant A_ (unknown
// ids as ACT_NONE, like apply_act): one switch per call site instead of one per element.
#define K44_WITH_ACT(act, ...)                                                                  \
    switch (act) {                                                                             \
    case ACT_RELU: { constexpr int A_ = ACT_RELU; __VA_ARGS__; } break;                         \
    case ACT_SIGMOID: { constexpr int A_ = ACT_SIGMOID; __VA_ARGS__; } break;                   \
    case ACT_SILU: { constexpr int A_ = ACT_SILU; __VA_ARGS__; } break;                         \
    case ACT_LEAKY: { constexpr int A_ = ACT_LEAKY; __VA_ARGS__; } break;                       \
    case ACT_GELU: { constexpr int A_ = ACT_GELU; __VA_ARGS__; } break;                         \
    default: { constexpr int A_ = ACT_NONE; __VA_ARGS__; } break;                               \
    }

struct GatherDotArgs {
    const __half *X;         // canvas base
    const uint64_t *seg;     // [rows][K] canvas element offset of each segment start
    const __half *W;         // [cout][K][n_batch][RPI][U] fp16, zero padded past S
    const __half *bias;      // [cout] or nullptr
    const uint16_t *cmap;    // [cout] or nullptr
    __half *Y;               // canvas + y_off
    const __half *R;         // canvas + res_off, or nullptr
    uint64_t step;           // canvas elements between consecutive positions of a segment
    uint32_t K, S, n_batch;  // segments per row, positions per segment, batches per segment
    uint32_t cluster;        // neurons per index row
    uint32_t cout;           // neurons (padded count)
    uint32_t out_stride;     // canvas elements between consecutive output neurons
    int act;
};

__device__ __forceinline__ void fma4(float (&acc)[4], float w, uint2 x) {
    const __half2 lo = *reinterpret_cast<const __half2 *>(&x.x);
    const __half2 hi = *reinterpret_cast<const __half2 *>(&x.y);
    const float2 a = __half22float2(lo), b = __half22float2(hi);
    acc[0] = fmaf(w, a.x, acc[0]);
    acc[1] = fmaf(w, a.y, acc[1]);
    acc[2] = fmaf(w, b.x, acc[2]);
    acc[3] = fmaf(w, b.y, acc[3]);
}

typedef unsigned int gd_u2 __attribute__((ext_vector_type(2)));
typedef unsigned int gd_u4 __attribute__((ext_vector_type(4)));

// Load of data the launch reads once.  NTX: a non-temporal load (the `nt` cache policy), for
// gathers from substrates far larger than the caches: measured on random 8 KiB segments of a
// 20 GB substrate, 6.86 TB/s against 6.2 TB/s with the default policy (equal on a 2 GB span).
template <bool NTX, typename T>
__device__ __forceinline__ T ld_once(const T *p) {
    if constexpr (NTX)
        return __builtin_nontemporal_load(p);
    else
        return *p;
}

template <int U, bool NTX>
__device__ __forceinline__ void load_weights(float (&w)[U], const __half *p) {
    static_assert(U == 2 || U == 4 || U % 8 == 0, "weights per lane: 2, 4 or a multiple of 8");
    if constexpr (U == 2) {
        const unsigned int v = ld_once<NTX>(reinterpret_cast<const unsigned int *>(p));
        const float2 f = __half22float2(*reinterpret_cast<const __half2 *>(&v));
        w[0] = f.x;
        w[1] = f.y;
    } else if constexpr (U == 4) {
        const gd_u2 v = ld_once<NTX>(reinterpret_cast<const gd_u2 *>(p));
        const __half *h = reinterpret_cast<const __half *>(&v);
#pragma unroll
        for (int u = 0; u < 4; ++u) w[u] = __half2float(h[u]);
    } else {
#pragma unroll
        for (int q = 0; q < U / 8; ++q) {
            const gd_u4 v = ld_once<NTX>(reinterpret_cast<const gd_u4 *>(p + 8 * q));
            const __half *h = reinterpret_cast<const __half *>(&v);
#pragma unroll
            for (int u = 0; u < 8; ++u) w[8 * q + u] = __half2float(h[u]);
        }
    }
}

// SLAB in {64, 128, 256}: tokens per wave.  U = rows per lane per batch.
// KSPLIT = 1: the 4 waves of a workgroup are 4 neurons.  KSPLIT = 4: the 4 waves share one
// neuron and take its segments round-robin (k = wave, wave + 4, ...); partial sums meet in LDS.
// Splitting keeps one short, fully parallel segment stream per wave when a neuron has only a
// few segments (the ultra-sparse regime), instead of serialising K load-wait-FMA phases.
// NTX: X rows and weights are read with non-temporal loads (see ld_once).
// MIS: segment starts may sit at any element (token-shifted taps of 1-D convolutions, the
// reference's `ch_base + dx`): each lane loads the two aligned 8-byte words around its 4 tokens
// and funnel-shifts them by the segment's misalignment (uniform per segment).  The second word
// reaches up to 3 elements past the last token used; the canvas carries slack for it.
template <int SLAB, int U, int KSPLIT, bool NTX, bool MIS = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8))) void k44_gather_dot_kernel(GatherDotArgs a) {
    constexpr int LPR = SLAB / 4;  // lanes per position row
    constexpr int RPI = 64 / LPR;  // rows per load instruction
    const int lane = (int)(threadIdx.x & 63u);
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const uint32_t j = KSPLIT == 1 ? blockIdx.x * 4u + (uint32_t)wave : blockIdx.x;
    if (j >= a.cout) return;  // uniform per wave (KSPLIT == 1) or per workgroup (KSPLIT == 4)
    const int g = lane / LPR, c = lane % LPR;
    const uint32_t slab0 = blockIdx.y * (uint32_t)SLAB;
    // Epilogue operands first: scalar loads that complete while the gathers are in flight.
    const uint32_t bias_w = scalar_word16(a.bias, a.W, j);
    const uint32_t cmap_w = scalar_word16(a.cmap, a.W, j);

    const kconst_u64 *seg = (const kconst_u64 *)a.seg + (uint64_t)(j / a.cluster) * a.K;
    const uint64_t batches = (uint64_t)a.K * a.n_batch;
    const __half *wl = a.W + (uint64_t)j * batches * (RPI * U) + g * U;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};

    // Row addresses: a wave-uniform row base (scalar) plus this lane's byte offset, so that each
    // load is one scalar-base + 32-bit-offset access and no 64-bit address lives in VGPRs.
    const uint32_t lane_off = 8u * (uint32_t)c;
    const uint64_t row_bytes = a.step * 2u;
    for (uint32_t k = KSPLIT == 1 ? 0u : (uint32_t)wave; k < a.K; k += KSPLIT) {
        uint64_t start = seg[k];
        uint32_t mis = 0u;  // elements past the 8-byte boundary below the segment start
        if constexpr (MIS) {
            mis = (uint32_t)(start & 3u);
            start -= mis;
        }
        const char *xseg = reinterpret_cast<const char *>(a.X + start + slab0);
        for (uint32_t b = 0; b < a.n_batch; ++b) {
            const uint32_t s0 = b * (uint32_t)(RPI * U) + (uint32_t)(g * U);
            gd_u2 x[U];
            if constexpr (MIS) {
                gd_u2 hi[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const uint32_t s = s0 + (uint32_t)u;
                    const char *p = xseg + (uint64_t)s * row_bytes + lane_off;
                    const bool in = s < a.S;
                    x[u] = in ? ld_once<NTX>(reinterpret_cast<const gd_u2 *>(p)) : gd_u2{0u, 0u};
                    hi[u] = in && mis ? ld_once<NTX>(reinterpret_cast<const gd_u2 *>(p + 8))
                                      : gd_u2{0u, 0u};
                }
                if (mis) {
                    // words d0..d3 of the lane's 8 elements; keep elements mis .. mis+3
                    const bool q = mis >= 2u, odd = (mis & 1u) != 0u;
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        const uint32_t a0 = q ? x[u].y : x[u].x, a1 = q ? hi[u].x : x[u].y,
                                       a2 = q ? hi[u].y : hi[u].x;
                        x[u].x = odd ? __builtin_amdgcn_alignbit(a1, a0, 16u) : a0;
                        x[u].y = odd ? __builtin_amdgcn_alignbit(a2, a1, 16u) : a1;
                    }
                }
            } else if ((b + 1u) * (uint32_t)(RPI * U) <= a.S) {  // whole batch inside the segment
#pragma unroll
                for (int u = 0; u < U; ++u)
                    x[u] = ld_once<NTX>(reinterpret_cast<const gd_u2 *>(
                        xseg + (uint64_t)(s0 + u) * row_bytes + lane_off));
            } else {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const uint32_t s = s0 + (uint32_t)u;
                    x[u] = s < a.S ? ld_once<NTX>(reinterpret_cast<const gd_u2 *>(
                                         xseg + (uint64_t)s * row_bytes + lane_off))
                                   : gd_u2{0u, 0u};
                }
            }
            const __half *wb = wl + ((uint64_t)k * a.n_batch + b) * (RPI * U);
            if constexpr (RPI == 1) {
                // One row per instruction: every lane needs the same U weights — scalar loads,
                // consumed straight from SGPRs.
                const kconst_u32 *ww = (const kconst_u32 *)wb;
#pragma unroll
                for (int u = 0; u < U; u += 2) {
                    const uint32_t pair = ww[u / 2];
                    const float2 wf = __half22float2(*reinterpret_cast<const __half2 *>(&pair));
                    fma4(acc, wf.x, make_uint2(x[u].x, x[u].y));
                    fma4(acc, wf.y, make_uint2(x[u + 1].x, x[u + 1].y));
                }
            } else {
                float w[U];
                load_weights<U, NTX>(w, wb);
#pragma unroll
                for (int u = 0; u < U; ++u) fma4(acc, w[u], make_uint2(x[u].x, x[u].y));
            }
        }
    }

#pragma unroll
    for (int off = LPR; off < 64; off <<= 1)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] += __shfl_xor(acc[t], off, 64);
    if constexpr (KSPLIT > 1) {
        __shared__ float part[KSPLIT][SLAB];
        if (g == 0) {
#pragma unroll
            for (int t = 0; t < 4; ++t) part[wave][4 * c + t] = acc[t];
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            float v = 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < KSPLIT; ++w2) v += part[w2][4 * c + t];
            acc[t] = v;
        }
    }
    if (g != 0) return;

    const uint64_t oj = a.cmap ? (uint64_t)half_of(cmap_w, j) : (uint64_t)j;
    const float bias =
        a.bias ? __half2float(__ushort_as_half((unsigned short)half_of(bias_w, j))) : 0.0f;
    if (a.cmap && oj == K44_CMAP_EMPTY) return;  // empty slot of a pattern-sorted tile: no output
    const uint64_t o = oj * a.out_stride + slab0 + 4u * (uint32_t)c;
    float r[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (a.R) {
        const gd_u2 rv = *reinterpret_cast<const gd_u2 *>(a.R + o);
        const __half *rh = reinterpret_cast<const __half *>(&rv);
#pragma unroll
        for (int t = 0; t < 4; ++t) r[t] = __half2float(rh[t]);
    }
    __half out[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const float v = acc[t] + bias;
        const float y = a.cmap ? apply_act(v + r[t], a.act) : apply_act(v, a.act) + r[t];
        out[t] = __float2half_rn(y);
    }
    *reinterpret_cast<gd_u2 *>(a.Y + o) = *reinterpret_cast<const gd_u2 *>(out);
}

// Variant with 8 tokens (16 bytes) per lane: half the load instructions per gathered byte of
// the 4-token kernel above, same weight layout (16 rows per batch, row = g*U + u).

__device__ __forceinline__ void fma8(float (&acc)[8], float w, gd_u4 x) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const unsigned int word = x[q];
        const float2 f = __half22float2(*reinterpret_cast<const __half2 *>(&word));
        acc[2 * q] = fmaf(w, f.x, acc[2 * q]);
        acc[2 * q + 1] = fmaf(w, f.y, acc[2 * q + 1]);
    }
}

// WL: the neuron's weights (K * n_batch * 16 <= GD_WL_MAX halves) are staged in LDS first, so no
// batch waits on a weight load from HBM (they are read once, never cache resident): cache-
// resident substrates (configs 1, 4) otherwise pay an HBM round trip per 16-row batch.

template <int SLAB, int KSPLIT, bool NTX, bool WL>
__global__ __launch_bounds__(256) void k44_gather_dot8_kernel(GatherDotArgs a) {
    constexpr int LPR = SLAB / 8;  // lanes per position row
    constexpr int RPI = 64 / LPR;  // rows per load instruction
    constexpr int U = 16 / RPI;    // loads in flight per lane (16 rows per batch)
    constexpr int NWL = WL ? (KSPLIT == 1 ? 4 : 1) : 0;
    __shared__ __attribute__((aligned(16))) __half wlds[NWL ? NWL : 1][NWL ? GD_WL_MAX : 8];
    const int lane = (int)(threadIdx.x & 63u);
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const uint32_t j = KSPLIT == 1 ? blockIdx.x * 4u + (uint32_t)wave : blockIdx.x;
    const uint64_t batches = (uint64_t)a.K * a.n_batch;
    if constexpr (WL) {
        // copy [batches][16] halves of this wave's (KSPLIT 1) / the workgroup's neuron
        const uint32_t n16 = (uint32_t)batches * 2u;  // 16-byte chunks
        const uint32_t jj = j < a.cout ? j : a.cout - 1u;
        const gd_u4 *src = reinterpret_cast<const gd_u4 *>(a.W + (uint64_t)jj * batches * 16u);
        gd_u4 *dst = reinterpret_cast<gd_u4 *>(&wlds[KSPLIT == 1 ? wave : 0][0]);
        const uint32_t t0 = KSPLIT == 1 ? (uint32_t)lane : threadIdx.x;
        const uint32_t tn = KSPLIT == 1 ? 64u : 256u;
        for (uint32_t q = t0; q < n16; q += tn) dst[q] = ld_once<NTX>(src + q);
        __syncthreads();
    }
    if (j >= a.cout) return;
    const int g = lane / LPR, c = lane % LPR;
    const uint32_t slab0 = blockIdx.y * (uint32_t)SLAB;
    const uint32_t bias_w = scalar_word16(a.bias, a.W, j);
    const uint32_t cmap_w = scalar_word16(a.cmap, a.W, j);

    const kconst_u64 *seg = (const kconst_u64 *)a.seg + (uint64_t)(j / a.cluster) * a.K;
    const __half *wl = WL ? &wlds[KSPLIT == 1 ? wave : 0][g * U]
                          : a.W + (uint64_t)j * batches * 16u + g * U;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};

    for (uint32_t k = KSPLIT == 1 ? 0u : (uint32_t)wave; k < a.K; k += KSPLIT) {
        const __half *xs = a.X + seg[k] + slab0 + 8u * (uint32_t)c;
        for (uint32_t b = 0; b < a.n_batch; ++b) {
            const uint32_t s0 = b * 16u + (uint32_t)(g * U);
            gd_u4 x[U];
            if ((b + 1u) * 16u <= a.S) {  // whole batch inside the segment
#pragma unroll
                for (int u = 0; u < U; ++u)
                    x[u] = ld_once<NTX>(reinterpret_cast<const gd_u4 *>(xs + (uint64_t)(s0 + u) * a.step));
            } else {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const uint32_t s = s0 + (uint32_t)u;
                    x[u] = s < a.S ? ld_once<NTX>(reinterpret_cast<const gd_u4 *>(xs + (uint64_t)s * a.step))
                                   : gd_u4{0u, 0u, 0u, 0u};
                }
            }
            float w[U];
            if constexpr (WL) {
                const __half *wp = wl + ((uint64_t)k * a.n_batch + b) * 16u;
#pragma unroll
                for (int u = 0; u < U; ++u) w[u] = __half2float(wp[u]);
            } else {
                load_weights<U, NTX>(w, wl + ((uint64_t)k * a.n_batch + b) * 16u);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) fma8(acc, w[u], x[u]);
        }
    }

#pragma unroll
    for (int off = LPR; off < 64; off <<= 1)
#pragma unroll
        for (int t = 0; t < 8; ++t) acc[t] += __shfl_xor(acc[t], off, 64);
    if constexpr (KSPLIT > 1) {
        __shared__ float part[KSPLIT][SLAB];
        if (g == 0) {
#pragma unroll
            for (int t = 0; t < 8; ++t) part[wave][8 * c + t] = acc[t];
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            float v = 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < KSPLIT; ++w2) v += part[w2][8 * c + t];
            acc[t] = v;
        }
    }
    if (g != 0) return;

    const uint64_t oj = a.cmap ? (uint64_t)half_of(cmap_w, j) : (uint64_t)j;
    const float bias =
        a.bias ? __half2float(__ushort_as_half((unsigned short)half_of(bias_w, j))) : 0.0f;
    if (a.cmap && oj == K44_CMAP_EMPTY) return;
    const uint64_t o = oj * a.out_stride + slab0 + 8u * (uint32_t)c;
    float r[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (a.R) {
        const gd_u4 rv = *reinterpret_cast<const gd_u4 *>(a.R + o);
        const __half *rh = reinterpret_cast<const __half *>(&rv);
#pragma unroll
        for (int t = 0; t < 8; ++t) r[t] = __half2float(rh[t]);
    }
    __half out[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const float v = acc[t] + bias;
        const float y = a.cmap ? apply_act(v + r[t], a.act) : apply_act(v, a.act) + r[t];
        out[t] = __float2half_rn(y);
    }
    *reinterpret_cast<gd_u4 *>(a.Y + o) = *reinterpret_cast<const gd_u4 *>(out);
}

// Streaming variant for waves whose gathers come from far beyond the caches (256-token slabs,
// 4 tokens per lane, no residual).  Measured on config 2's pattern: the write of each neuron's
// 512-byte output row, interleaved with the random gathers, costs ~15 % of the kernel (HBM
// read/write turnaround: 308 us of pure gathers, 366 us with the rows written as they are
// done, 320 us when they are written in one burst at the end).  So a workgroup owns NPW
// neurons of one slab, keeps their finished fp16 rows in LDS (NPW x 512 B) and writes them
// after its last gather.  Wave w takes neurons w, w + WAVES, ...; its work is the flat list of
// (neuron, segment, 16-row batch) steps, two steps in flight (the loads of step t+1 are issued
// before the FMAs of step t).  Per neuron the accumulation order is that of
// k44_gather_dot_kernel<256, 16, 1>: segments, batches and rows in order, one FMA chain — the
// two kernels give bit-identical outputs.  Weights are scalar loads (every lane needs the same
// 16 per batch).
template <int NPW, int WAVES, bool NTX>
__global__ __launch_bounds__(WAVES * 64) void k44_gather_stream_kernel(GatherDotArgs a) {
    constexpr int U = 16;
    static_assert(NPW % WAVES == 0, "whole neuron slots per wave");
    __shared__ gd_u2 orow[NPW][64];
    const int lane = (int)(threadIdx.x & 63u);
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const uint32_t j0 = blockIdx.x * (uint32_t)NPW;
    const uint32_t slab0 = blockIdx.y * 256u;
    const uint32_t lane_off = 8u * (uint32_t)lane;
    const uint64_t row_bytes = a.step * 2u;
    // Neurons of this wave: j0 + wave + i*WAVES for i < n_mine (the last workgroup may be short).
    const uint32_t n_here = min((uint32_t)NPW, a.cout - j0);
    const uint32_t n_mine = n_here > (uint32_t)wave ? (n_here - (uint32_t)wave + WAVES - 1u) / WAVES : 0u;
    const uint32_t per_neuron = a.K * a.n_batch;
    const uint32_t total = n_mine * per_neuron;

    // Step t -> (neuron slot i, segment k, batch b) by running counters, advanced per step.
    struct Cursor {
        uint32_t i, k, b;
    };
    auto advance = [&](Cursor &c) {
        if (++c.b == a.n_batch) {
            c.b = 0;
            if (++c.k == a.K) {
                c.k = 0;
                ++c.i;
            }
        }
    };
    // issue(): the step's rows and its 16 weights (scalar loads), one step ahead of consume().
    auto issue = [&](const Cursor &c, gd_u2 (&x)[U], uint32_t (&wv)[U / 2]) {
        const uint32_t j = j0 + (uint32_t)wave + c.i * WAVES;
        const kconst_u32 *ww =
            (const kconst_u32 *)(a.W + (((uint64_t)j * a.K + c.k) * a.n_batch + c.b) * U);
#pragma unroll
        for (int u = 0; u < U / 2; ++u) wv[u] = ww[u];
        const kconst_u64 *seg = (const kconst_u64 *)a.seg + (uint64_t)(j / a.cluster) * a.K;
        const char *xseg = reinterpret_cast<const char *>(a.X + seg[c.k] + slab0);
        const uint32_t s0 = c.b * (uint32_t)U;
        if (s0 + (uint32_t)U <= a.S) {
#pragma unroll
            for (int u = 0; u < U; ++u)
                x[u] = ld_once<NTX>(reinterpret_cast<const gd_u2 *>(
                    xseg + (uint64_t)(s0 + u) * row_bytes + lane_off));
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t s = s0 + (uint32_t)u;
                x[u] = s < a.S ? ld_once<NTX>(reinterpret_cast<const gd_u2 *>(
                                     xseg + (uint64_t)s * row_bytes + lane_off))
                               : gd_u2{0u, 0u};
            }
        }
    };
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto consume = [&](const Cursor &c, const gd_u2 (&x)[U], const uint32_t (&wv)[U / 2]) {
        const uint32_t j = j0 + (uint32_t)wave + c.i * WAVES;
#pragma unroll
        for (int u = 0; u < U; u += 2) {
            const uint32_t pair = wv[u / 2];
            const float2 wf = __half22float2(*reinterpret_cast<const __half2 *>(&pair));
            fma4(acc, wf.x, make_uint2(x[u].x, x[u].y));
            fma4(acc, wf.y, make_uint2(x[u + 1].x, x[u + 1].y));
        }
        if (c.k + 1u == a.K && c.b + 1u == a.n_batch) {  // neuron done: fused epilogue into LDS
            const float bias =
                a.bias ? __half2float(__ushort_as_half((unsigned short)half_of(scalar_word16(a.bias, a.W, j), j)))
                       : 0.0f;
            __half out[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                out[t] = __float2half_rn(apply_act(acc[t] + bias, a.act));
                acc[t] = 0.0f;
            }
            orow[(uint32_t)wave + c.i * WAVES][lane] = *reinterpret_cast<const gd_u2 *>(out);
        }
    };

    gd_u2 xa[U], xb[U];
    uint32_t wa[U / 2], wb[U / 2];
    Cursor ca{0u, 0u, 0u};
    if (total) issue(ca, xa, wa);
    for (uint32_t t = 0; t < total; t += 2) {
        Cursor cb = ca;
        advance(cb);
        if (t + 1u < total) issue(cb, xb, wb);
        consume(ca, xa, wa);
        if (t + 1u >= total) break;
        ca = cb;
        advance(ca);
        if (t + 2u < total) issue(ca, xa, wa);
        consume(cb, xb, wb);
    }
    __syncthreads();
    // Burst write of the finished rows: wave w writes rows w, w + WAVES, ... (512 B each).
    for (uint32_t l = (uint32_t)wave; l < n_here; l += WAVES) {
        const uint32_t j = j0 + l;
        const uint64_t oj = a.cmap ? (uint64_t)half_of(scalar_word16(a.cmap, a.W, j), j) : (uint64_t)j;
        if (a.cmap && oj == K44_CMAP_EMPTY) continue;
        gd_u2 *dst = reinterpret_cast<gd_u2 *>(a.Y + oj * a.out_stride + slab0) + lane;
        if constexpr (NTX)
            __builtin_nontemporal_store(orow[l][lane], dst);
        else
            *dst = orow[l][lane];
    }
}

// Synthetic substrate: X[pos][t] = fp16_rne((int32(h >> 40) - 2^23) * 2^-23) with
// h = splitmix64(((pos << 20) | t) ^ splitmix64(seed)); tokens t >= valid are zero.
__host__ __device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    uint64_t z = x + 0x9e3779b97f4a7c15ULL;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

}  // namespace k44dev
