// Translation unit of the 1-D token ops (see k44_aux.hpp for their semantics).
#include "k44_aux.hpp"
#include "k44_gather_dot.hpp"
#include "k44_sumsq.hpp"

namespace k44dev {

// Workgroup = OCT token octets (8 consecutive tokens = one 16-byte column chunk each) x
// 256/OCT channel lanes: every lane sums squares down its channel stripe with 8 loads in flight
// (OCT lanes side by side read 16*OCT contiguous bytes of a channel row), the lanes of an octet
// reduce (shuffles, then the 4 waves in LDS), and the workgroup writes channel slice blockIdx.y
// of its tokens.  The sums of squares are exact (k44_sumsq.hpp): the same bits whatever the
// grouping, so a norm whose sums were assembled elsewhere (slots: the per-tile sums of the waves
// that produced x, added here) gives this kernel's output exactly; with slots the sum pass over
// all D channels is skipped.  Small token counts (decode) use OCT = 1 and several slices
// per token chunk, each recomputing the (cache-resident) sum, so the grid still fills the chip.
// RF > 0 (decode slices of one channel per thread): the decode token shift of the output
// follows in the same thread — y2 = mu[c][0]*y + sum_i mu[c][i]*state[c][i-1][t], state shifted
// in place, with the arithmetic of k44_token_shift_decode_kernel (bit-identical); the grid
// then covers every octet of the stride, octets without requests writing zeros to y2 only.
template <int OCT, uint32_t RF>
__global__ __launch_bounds__(256) void k44_rmsnorm_kernel(__half *__restrict__ y,
                                                          const __half *__restrict__ x,
                                                          const __half *__restrict__ gamma,
                                                          uint32_t D, uint32_t stride, float eps,
                                                          uint32_t cslice, RmsShift sh,
                                                          const uint64_t *__restrict__ slots,
                                                          uint32_t n_slots) {
    constexpr uint32_t CL = 256u / OCT;  // channel lanes
    __shared__ SumSq part[4][OCT * 8];
    __shared__ float inv_s[OCT * 8];
    const uint32_t oct = threadIdx.x % OCT, lane_c = threadIdx.x / OCT;
    const uint32_t t0 = (blockIdx.x * OCT + oct) * 8u;
    // Slices of at most one channel per thread (decode): the thread's own channel and its gamma
    // are loaded with the sum's loads instead of after the reduction.
    const uint32_t c_end = min(D, (blockIdx.y + 1u) * cslice);
    const bool one = cslice <= CL;
    const uint32_t c_own = blockIdx.y * cslice + lane_c;
    uint4 xo = {0u, 0u, 0u, 0u};
    // Fused token shift: octets without requests only write zeros; the mixing weights and the
    // state of the thread's channel are loaded here too.
    if constexpr (RF > 0u) {
        // the shift's kernel arguments are read before the branch (one round trip, not two)
        asm volatile("" ::"s"(sh.tokens), "s"(sh.y2), "s"(sh.mu), "s"(sh.state));
        if (t0 >= sh.tokens) {
            if (c_own < c_end)
                *reinterpret_cast<uint4 *>(sh.y2 + (uint64_t)c_own * stride + t0) =
                    uint4{0u, 0u, 0u, 0u};
            return;  // uniform: one octet per workgroup
        }
    }
    // Every lane loads (the last channel of the slice stands in for lanes past it, whose
    // results are not written; slices of several channels per thread do not use these), and
    // the values are held opaque until after the sum's loads: a load under a branch, or one
    // converted right away, makes the compiler wait for it before the sum's loads are issued.
    // Without gamma, x stands in for it (unused).
    uint32_t gbits, mbits[RF > 0u ? RF : 1u];
    uint4 sv[RF > 1u ? RF - 1u : 1u];
    {
        const uint32_t cc = c_own < c_end ? c_own : c_end - 1u;
        xo = *reinterpret_cast<const uint4 *>(x + (uint64_t)cc * stride + t0);
        gbits = reinterpret_cast<const uint16_t *>(gamma ? gamma : x)[cc];
        if constexpr (RF > 0u) {
            const uint16_t *m = reinterpret_cast<const uint16_t *>(sh.mu) + (uint64_t)cc * RF;
#pragma unroll
            for (uint32_t i = 0; i < RF; ++i) mbits[i] = m[i];
            const __half *st = sh.state + (uint64_t)cc * (RF - 1u) * 64u + t0;
#pragma unroll
            for (uint32_t i = 1; i < RF; ++i)
                sv[i - 1] = *reinterpret_cast<const uint4 *>(st + (i - 1u) * 64u);
        }
    }
    SumSq ss[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) ss[k] = sumsq_zero();
    uint32_t c = slots ? D : lane_c;  // (uniform) scales from the producers' sums: no sum pass
    auto add8 = [&](const uint4 &v) {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 8; ++k) sumsq_add(ss[k], w[k >> 1] >> (16 * (k & 1)));
    };
    for (; c + 7u * CL < D; c += 8u * CL) {
        uint4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            v[u] = *reinterpret_cast<const uint4 *>(x + (uint64_t)(c + u * CL) * stride + t0);
#pragma unroll
        for (int u = 0; u < 8; ++u) add8(v[u]);
    }
    for (; c < D; c += CL) add8(*reinterpret_cast<const uint4 *>(x + (uint64_t)c * stride + t0));
    // the own-channel values become visible to the compiler only here
    asm volatile("" : "+v"(xo.x), "+v"(xo.y), "+v"(xo.z), "+v"(xo.w), "+v"(gbits));
    if constexpr (RF > 0u) {
#pragma unroll
        for (uint32_t i = 0; i < RF; ++i) asm volatile("" : "+v"(mbits[i]));
#pragma unroll
        for (uint32_t i = 1; i < RF; ++i)
            asm volatile("" : "+v"(sv[i - 1].x), "+v"(sv[i - 1].y), "+v"(sv[i - 1].z), "+v"(sv[i - 1].w));
    }
    if (slots) {
        // one octet per workgroup (decode): its 8 tokens' scales from the producers' slots
        __shared__ uint4 spart[4][8];
        __shared__ float sinv[8];
        rms_inv_from_slots<8u>(slots, n_slots, blockIdx.x * 8u, D, eps, spart, sinv);
        if (threadIdx.x < 8u) inv_s[threadIdx.x] = sinv[threadIdx.x];
    } else {
        // Per-token sums of the CL channel lanes: transposed through LDS ([token][lane], carries
        // propagated), then thread (token k, part p) adds 8 lanes, the parts of a token meet
        // by shuffles within the wave and the 4 waves in LDS (exact: any order).
        constexpr uint32_t TK = OCT * 8u;  // tokens of the workgroup
        __shared__ uint4 tr[TK][CL];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const SumSq q = sumsq_norm(ss[k]);
            tr[oct * 8u + k][lane_c] = uint4{(uint32_t)q.l0, (uint32_t)q.l1, (uint32_t)q.l2, q.sp};
        }
        __syncthreads();
        const uint32_t k = threadIdx.x % TK, pp = threadIdx.x / TK;
        SumSq a = sumsq_zero();
#pragma unroll
        for (uint32_t j = 0; j < 8u; ++j) {
            const uint4 v = tr[k][pp * 8u + j];
            a.l0 += v.x;
            a.l1 += v.y;
            a.l2 += v.z;
            a.sp |= v.w;
        }
        a = sumsq_wave_reduce(a, (int)TK);
        const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
        if (lane < TK) part[wave][lane] = a;
        __syncthreads();
        if (threadIdx.x < TK) {
            SumSq t = part[0][threadIdx.x];
            sumsq_merge(t, part[1][threadIdx.x]);
            sumsq_merge(t, part[2][threadIdx.x]);
            sumsq_merge(t, part[3][threadIdx.x]);
            inv_s[threadIdx.x] = rms_inv(t, D, eps);
        }
    }
    __syncthreads();
    float inv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) inv[k] = inv_s[oct * 8u + k];
    if (one) {
        if (c_own < c_end) {
            const __half *h = reinterpret_cast<const __half *>(&xo);
            uint4 o;
            __half *oh = reinterpret_cast<__half *>(&o);
            const float go = gamma ? __half2float(__ushort_as_half((unsigned short)gbits)) : 1.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k) oh[k] = norm_scale(h[k], inv[k], go);
            if (RF == 0u || t0 < sh.tokens)
                *reinterpret_cast<uint4 *>(y + (uint64_t)c_own * stride + t0) = o;
            if constexpr (RF > 0u) {
                __half *st = sh.state + (uint64_t)c_own * (RF - 1u) * 64u + t0;
                uint4 o2;
                __half *yh = reinterpret_cast<__half *>(&o2);
                uint4 nsv[RF > 1u ? RF - 1u : 1u];
#pragma unroll
                for (uint32_t i = 1; i < RF; ++i) nsv[i - 1] = sv[i - 1];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    if (t0 + (uint32_t)k >= sh.tokens) {
                        yh[k] = __float2half_rn(0.0f);
                        continue;
                    }
                    float mw[RF];
#pragma unroll
                    for (uint32_t i = 0; i < RF; ++i)
                        mw[i] = __half2float(__ushort_as_half((unsigned short)mbits[i]));
                    float acc = mw[0] * __half2float(oh[k]);
#pragma unroll
                    for (uint32_t i = 1; i < RF; ++i)
                        acc = fmaf(mw[i], __half2float(reinterpret_cast<const __half *>(&sv[i - 1])[k]), acc);
                    yh[k] = f16_of(acc);
#pragma unroll
                    for (uint32_t i = RF - 1u; i > 1u; --i)
                        reinterpret_cast<__half *>(&nsv[i - 1])[k] =
                            reinterpret_cast<const __half *>(&sv[i - 2])[k];
                    if (RF > 1u) reinterpret_cast<__half *>(&nsv[0])[k] = oh[k];
                }
#pragma unroll
                for (uint32_t i = 1; i < RF; ++i)
                    *reinterpret_cast<uint4 *>(st + (i - 1u) * 64u) = nsv[i - 1];
                *reinterpret_cast<uint4 *>(sh.y2 + (uint64_t)c_own * stride + t0) = o2;
            }
        }
        return;
    }
    for (c = blockIdx.y * cslice + lane_c; c < c_end; c += CL) {
        const uint4 v = *reinterpret_cast<const uint4 *>(x + (uint64_t)c * stride + t0);
        const __half *h = reinterpret_cast<const __half *>(&v);
        const float g = gamma ? __half2float(gamma[c]) : 1.0f;
        uint4 o;
        __half *oh = reinterpret_cast<__half *>(&o);
#pragma unroll
        for (int k = 0; k < 8; ++k) oh[k] = norm_scale(h[k], inv[k], g);
        *reinterpret_cast<uint4 *>(y + (uint64_t)c * stride + t0) = o;
    }
}

// Wide token counts (prefill): workgroup = 4 token octets (32 tokens, 64-byte row runs) x 256
// channel lanes (1024 threads), one workgroup per 32 tokens.  A thread loads its CPT channels
// (lane, lane + 256, ...) and their gammas once, keeps them in registers for the sum of squares
// and the scaled store: the input is read once (the narrower kernel above reads it twice).  All
// loads are issued together, without branches around them (channels >= D read row D - 1 and
// drop it): a load under a divergent branch, or one placed among the stores, makes the compiler
// wait for every access before it, stores included.  Sums meet by shuffles within a wave, then
// across the 16 waves in LDS in wave order.
template <int CPT>
__global__ __launch_bounds__(1024) void k44_rmsnorm_regs_kernel(__half *__restrict__ y,
                                                                const __half *__restrict__ x,
                                                                const __half *__restrict__ gamma,
                                                                uint32_t D, uint32_t stride,
                                                                float eps) {
    constexpr uint32_t OCT = 4u, CL = 256u;
    __shared__ float part[16][OCT * 8];
    __shared__ float inv_s[OCT * 8];
    const uint32_t oct = threadIdx.x % OCT, lane_c = threadIdx.x / OCT;
    const uint32_t t0 = (blockIdx.x * OCT + oct) * 8u;
    // gamma bits one per register (CPT <= 8; 16 channels a thread load theirs at the store);
    // without gamma x's first row stands in for it, unused
    constexpr int GR = CPT <= 8 ? CPT : 1;
    uint4 v[CPT];
    uint32_t gv[GR];
    const uint16_t *g16 = reinterpret_cast<const uint16_t *>(gamma ? gamma : x);
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const uint32_t c = lane_c + (uint32_t)u * CL;
        const uint32_t cc = c < D ? c : D - 1u;
        const uint4 t = *reinterpret_cast<const uint4 *>(x + (uint64_t)cc * stride + t0);
        v[u] = c < D ? t : uint4{0u, 0u, 0u, 0u};
        if constexpr (CPT <= 8) gv[u] = g16[cc];
    }
    float ss[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const __half *h = reinterpret_cast<const __half *>(&v[u]);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float f = __half2float(h[k]);
            ss[k] = fmaf(f, f, ss[k]);
        }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
        for (uint32_t m = OCT; m < 64u; m <<= 1) ss[k] += __shfl_xor(ss[k], (int)m, 64);
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    if (lane < OCT) {
#pragma unroll
        for (int k = 0; k < 8; ++k) part[wave][lane * 8u + k] = ss[k];
    }
    __syncthreads();
    if (threadIdx.x < OCT * 8u) {  // one total per (octet, token), the waves added in order
        float t = part[0][threadIdx.x];
        for (int w = 1; w < 16; ++w) t += part[w][threadIdx.x];
        inv_s[threadIdx.x] = rsqrtf(t / (float)D + eps);
    }
    __syncthreads();
    float inv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) inv[k] = inv_s[oct * 8u + k];
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const uint32_t c = lane_c + (uint32_t)u * CL;
        if (c >= D) break;
        const __half *h = reinterpret_cast<const __half *>(&v[u]);
        float g = 1.0f;
        if constexpr (CPT <= 8) {
            if (gamma) g = __half2float(__ushort_as_half((unsigned short)gv[u]));
        } else if (gamma) {
            g = __half2float(gamma[c]);
        }
        uint4 o;
        __half *oh = reinterpret_cast<__half *>(&o);
#pragma unroll
        for (int k = 0; k < 8; ++k) oh[k] = norm_scale(h[k], inv[k], g);
        *reinterpret_cast<uint4 *>(y + (uint64_t)c * stride + t0) = o;
    }
}

// Prefill RMSNorm with the token shift of its output fused (k44_rmsnorm_regs_kernel followed by
// k44_token_shift_prefill_kernel, the same operations in the same order, so the same values).
// The workgroup of 32 tokens also sums the squares of the HK = 4 tokens before its block (the
// taps reach RF - 1 <= 4 tokens back), reduced in the order of the workgroup that owns them
// (same channels per thread, same shuffle tree, waves in order), so their norms are that
// workgroup's; the shift of octets 1..3 takes the previous octet's normalized values from the
// neighbouring lane (thread = 4 * channel lane + octet), octet 0 from those 4 tokens.  Writes the norm output y, the shift output y2 and the state
// block (each request's last RF-1 normalized tokens).  Token t of the block is at request
// position t % seq_len; tap i applies when i <= that position.
template <int CPT, uint32_t RF>
__global__ __launch_bounds__(1024) void k44_rmsnorm_shift_prefill_kernel(
    __half *__restrict__ y, const __half *__restrict__ x, const __half *__restrict__ gamma,
    uint32_t D, uint32_t stride, float eps, __half *__restrict__ y2,
    const __half *__restrict__ mu, __half *__restrict__ state, uint32_t seq_len) {
    constexpr uint32_t OCT = 4u, CL = 256u;
    // tokens before the block the taps reach: RF - 1, rounded up to a 4-token (8-byte) load
    static_assert(RF >= 1u && RF <= 5u, "the registers hold the 4 tokens before the block");
    constexpr uint32_t HK = RF <= 1u ? 0u : 4u;
    constexpr uint32_t HS = HK ? HK : 1u;
    __shared__ float part[16][OCT * 8 + HS];
    __shared__ float inv_s[OCT * 8 + HS];
    __shared__ __half mus[2048u * RF], gms[2048u];  // mixing weights and gamma (D <= 2048)
    const uint32_t oct = threadIdx.x % OCT, lane_c = threadIdx.x / OCT;
    const uint32_t t0 = (blockIdx.x * OCT + oct) * 8u;
    const bool halo = HK && oct == 0u && t0 >= 8u;
    // Every lane issues every load, without branches (a load under a divergent branch makes the
    // compiler wait for all accesses before it): channels >= D read row D - 1, lanes without a
    // halo read the 4 tokens at t0, and both are replaced by zeros after the load.
    uint4 v[CPT];
    uint32_t hv[CPT][HS / 2];  // the HK tokens before t0 (octet 0 lanes)
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const uint32_t c = lane_c + (uint32_t)u * CL;
        const bool live = c < D;
        const __half *xr = x + (uint64_t)(live ? c : D - 1u) * stride;
        const uint4 t = *reinterpret_cast<const uint4 *>(xr + t0);
        v[u] = live ? t : uint4{0u, 0u, 0u, 0u};
#pragma unroll
        for (uint32_t j = 0; j < HS / 2; ++j) hv[u][j] = 0u;
        if constexpr (HK == 4u) {
            const uint2 hx = *reinterpret_cast<const uint2 *>(xr + (halo ? t0 - 4u : t0));
            hv[u][0] = halo && live ? hx.x : 0u;
            hv[u][1] = halo && live ? hx.y : 0u;
        }
    }
    // the channels' mixing weights and gamma, staged in LDS (visible after the barrier below);
    // all loads issued before the first LDS write, indices clamped rather than branched around
    constexpr uint32_t NMU = (2048u * RF + 1023u) / 1024u, NGM = 2u;
    uint32_t mv[NMU], gmv[NGM];
    const uint16_t *mu16 = reinterpret_cast<const uint16_t *>(mu);
    const uint16_t *g16 = reinterpret_cast<const uint16_t *>(gamma);
#pragma unroll
    for (uint32_t j = 0; j < NMU; ++j) {
        const uint32_t e = threadIdx.x + j * 1024u;
        mv[j] = mu16[e < D * RF ? e : 0u];
    }
#pragma unroll
    for (uint32_t j = 0; j < NGM; ++j) {
        const uint32_t e = threadIdx.x + j * 1024u;
        gmv[j] = g16 ? (uint32_t)g16[e < D ? e : 0u] : 0x3C00u;  // fp16 1.0 without gamma
    }
#pragma unroll
    for (uint32_t j = 0; j < NMU; ++j) {
        const uint32_t e = threadIdx.x + j * 1024u;
        if (e < D * RF) mus[e] = __ushort_as_half((unsigned short)mv[j]);
    }
#pragma unroll
    for (uint32_t j = 0; j < NGM; ++j) {
        const uint32_t e = threadIdx.x + j * 1024u;
        if (e < D) gms[e] = __ushort_as_half((unsigned short)gmv[j]);
    }
    float ss[8] = {0, 0, 0, 0, 0, 0, 0, 0}, sh[HS];
#pragma unroll
    for (uint32_t k = 0; k < HS; ++k) sh[k] = 0.0f;
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const __half *h = reinterpret_cast<const __half *>(&v[u]);
        const __half *hh = reinterpret_cast<const __half *>(&hv[u][0]);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float f = __half2float(h[k]);
            ss[k] = fmaf(f, f, ss[k]);
        }
#pragma unroll
        for (uint32_t k = 0; k < HK; ++k) {
            const float fh = __half2float(hh[k]);
            sh[k] = fmaf(fh, fh, sh[k]);
        }
    }
#pragma unroll
    for (uint32_t m = OCT; m < 64u; m <<= 1) {
#pragma unroll
        for (int k = 0; k < 8; ++k) ss[k] += __shfl_xor(ss[k], (int)m, 64);
#pragma unroll
        for (uint32_t k = 0; k < HK; ++k) sh[k] += __shfl_xor(sh[k], (int)m, 64);
    }
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    if (lane < OCT) {
#pragma unroll
        for (int k = 0; k < 8; ++k) part[wave][lane * 8u + k] = ss[k];
    }
    if (HK && lane == 0u) {
#pragma unroll
        for (uint32_t k = 0; k < HK; ++k) part[wave][OCT * 8u + k] = sh[k];
    }
    __syncthreads();
    if (threadIdx.x < OCT * 8u + HK) {  // one total per token (block octets, then those before)
        float t = part[0][threadIdx.x];
        for (int w = 1; w < 16; ++w) t += part[w][threadIdx.x];
        inv_s[threadIdx.x] = rsqrtf(t / (float)D + eps);
    }
    __syncthreads();
    // requests are multiples of 8 tokens: an octet lies in one request, positions pos0 + k
    const uint32_t pos0 = t0 % seq_len;
    const bool near_end = pos0 + 7u + RF > seq_len;
    const int src_lane = (int)((lane + 63u) & 63u);  // octet - 1, same channel lane
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const uint32_t c = lane_c + (uint32_t)u * CL;
        const bool live = c < D;
        const float g = live ? __half2float(gms[c]) : 1.0f;
        const __half *h = reinterpret_cast<const __half *>(&v[u]);
        uint4 o;
        __half *oh = reinterpret_cast<__half *>(&o);
#pragma unroll
        for (int k = 0; k < 8; ++k) oh[k] = norm_scale(h[k], inv_s[oct * 8u + k], g);
        // the 8 tokens before: the neighbouring lane's normalized octet (every lane shuffles);
        // octet 0: its own HK tokens normalized, the rest unused by the taps
        uint4 pv;
        pv.x = (uint32_t)__shfl((int)o.x, src_lane, 64);
        pv.y = (uint32_t)__shfl((int)o.y, src_lane, 64);
        pv.z = (uint32_t)__shfl((int)o.z, src_lane, 64);
        pv.w = (uint32_t)__shfl((int)o.w, src_lane, 64);
        if (oct == 0u) {
            pv = uint4{0u, 0u, 0u, 0u};
            if (halo) {
                const __half *hh = reinterpret_cast<const __half *>(&hv[u][0]);
                __half *ph = reinterpret_cast<__half *>(&pv);
#pragma unroll
                for (uint32_t k = 0; k < HK; ++k)
                    ph[8u - HK + k] = norm_scale(hh[k], inv_s[OCT * 8u + k], g);
            }
        }
        if (!live) continue;
        *reinterpret_cast<uint4 *>(y + (uint64_t)c * stride + t0) = o;
        float m[RF];
#pragma unroll
        for (uint32_t i = 0; i < RF; ++i) m[i] = __half2float(mus[c * RF + i]);
        float w[16];  // w[8 + k] = u[t0 + k], w[k] = u[t0 - 8 + k]
        const __half *hp = reinterpret_cast<const __half *>(&pv);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            w[8 + k] = __half2float(oh[k]);
            w[k] = __half2float(hp[k]);
        }
        uint4 s;
        __half *sh2 = reinterpret_cast<__half *>(&s);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            float acc = m[0] * w[8 + k];
#pragma unroll
            for (uint32_t i = 1; i < RF; ++i)
                if (i <= pos0 + (uint32_t)k) acc = fmaf(m[i], w[8 + k - i], acc);
            sh2[k] = f16_of(acc);
        }
        *reinterpret_cast<uint4 *>(y2 + (uint64_t)c * stride + t0) = s;
        if (RF > 1u && state && near_end) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (pos0 + (uint32_t)k + RF > seq_len) {
                    const uint32_t back = seq_len - 1u - (pos0 + (uint32_t)k);  // 0 = newest
                    state[((uint64_t)c * (RF - 1u) + back) * 64u + (t0 + (uint32_t)k) / seq_len] =
                        oh[k];
                }
            }
        }
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

// m = a * (b * c) with the two commands' roundings: fp16(a * fp16(b * c)).  Products of two
// fp16 values are exact in fp32, so each rounding is the one multiply command's.  No restrict:
// the output may be one of the operands (same element, same thread).
__global__ __launch_bounds__(256) void k44_mul3_kernel(__half *y, const __half *a,
                                                       const __half *b, const __half *c,
                                                       uint64_t n8) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < n8;
         i += (uint64_t)gridDim.x * 256u) {
        const uint4 va = reinterpret_cast<const uint4 *>(a)[i];
        const uint4 vb = reinterpret_cast<const uint4 *>(b)[i];
        const uint4 vc = reinterpret_cast<const uint4 *>(c)[i];
        const __half *ha = reinterpret_cast<const __half *>(&va);
        const __half *hb = reinterpret_cast<const __half *>(&vb);
        const __half *hc = reinterpret_cast<const __half *>(&vc);
        uint4 o;
        __half *ho = reinterpret_cast<__half *>(&o);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const __half bc = __float2half_rn(__half2float(hb[k]) * __half2float(hc[k]));
            ho[k] = __float2half_rn(__half2float(ha[k]) * __half2float(bc));
        }
        reinterpret_cast<uint4 *>(y)[i] = o;
    }
}

// Prefill: thread = (TS_CPC channels c0 + j, c0 = (blockIdx.y + k*gridDim.y) * TS_CPC, 8
// consecutive tokens), with the 8 tokens before them in registers (RF - 1 <= 8), so every tap
// is a register read; the loads of all TS_CPC channels are issued before the first is used.
// The receptive field is a template parameter (the taps unroll without per-tap tests of rf).
// Token t is at position pos = t % seq_len of its request; tap i applies when i <= pos.
// State block of channel c: state[(c*(RF-1) + i)*64 + r] = input of request r, i+1 tokens back.
constexpr uint32_t TS_CPC = 4;
template <uint32_t RF>
__global__ __launch_bounds__(256) void k44_token_shift_prefill_kernel(
    __half *__restrict__ y, const __half *__restrict__ x, const __half *__restrict__ mu,
    __half *__restrict__ state, uint32_t D, uint32_t stride, uint32_t tokens, uint32_t seq_len) {
    const uint32_t chunk = blockIdx.x * 256u + threadIdx.x;
    const uint32_t t0 = chunk * 8u;
    if (t0 >= stride) return;
    uint32_t pos_k[8];  // request position of each of the 8 tokens
    {
        uint32_t pos = t0 % seq_len;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            pos_k[k] = pos;
            pos = pos + 1u == seq_len ? 0u : pos + 1u;
        }
    }
    // State entries fall in this chunk only near a request's end.
    bool near_end = false;
#pragma unroll
    for (int k = 0; k < 8; ++k) near_end = near_end || pos_k[k] + RF > seq_len;
    for (uint32_t c0 = blockIdx.y * TS_CPC; c0 < D; c0 += gridDim.y * TS_CPC) {
        // Every load of the channel block is issued before any value is used, without
        // branches around them (the first octet reads its own tokens as the "previous" ones and
        // drops them, channels past D read row D - 1): a load under a divergent branch, or one
        // converted right away, would be waited for before the next is issued.
        uint4 cur[TS_CPC], prv[TS_CPC];
        uint32_t mb[TS_CPC][RF];
        const uint16_t *mu16 = reinterpret_cast<const uint16_t *>(mu);
#pragma unroll
        for (uint32_t j = 0; j < TS_CPC; ++j) {
            const uint32_t c = c0 + j < D ? c0 + j : D - 1u;
            const __half *xr = x + (uint64_t)c * stride;
            cur[j] = *reinterpret_cast<const uint4 *>(xr + t0);
            prv[j] = *reinterpret_cast<const uint4 *>(xr + (t0 ? t0 - 8u : t0));
#pragma unroll
            for (uint32_t i = 0; i < RF; ++i) mb[j][i] = mu16[(uint64_t)c * RF + i];
        }
#pragma unroll
        for (uint32_t j = 0; j < TS_CPC; ++j) {
            const uint32_t c = c0 + j;
            if (c >= D) break;
            float m[RF];
#pragma unroll
            for (uint32_t i = 0; i < RF; ++i)
                m[i] = __half2float(__ushort_as_half((unsigned short)mb[j][i]));
            float w[16];  // w[8 + k] = x[t0 + k], w[k] = x[t0 - 8 + k] (zero before the stride)
            const __half *hc = reinterpret_cast<const __half *>(&cur[j]);
            const __half *hp = reinterpret_cast<const __half *>(&prv[j]);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                w[8 + k] = __half2float(hc[k]);
                w[k] = t0 ? __half2float(hp[k]) : 0.0f;
            }
            uint4 o;
            __half *oh = reinterpret_cast<__half *>(&o);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                float acc = 0.0f;
                if (t0 + (uint32_t)k < tokens) {
                    acc = m[0] * w[8 + k];
#pragma unroll
                    for (uint32_t i = 1; i < RF; ++i)
                        if (i <= pos_k[k]) acc = fmaf(m[i], w[8 + k - i], acc);
                }
                oh[k] = f16_of(acc);
            }
            *reinterpret_cast<uint4 *>(y + (uint64_t)c * stride + t0) = o;
            if (RF > 1u && state && near_end) {  // last RF-1 tokens of the request -> state
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const uint32_t t = t0 + (uint32_t)k;
                    if (t < tokens && pos_k[k] + RF > seq_len) {
                        const uint32_t back = seq_len - 1u - pos_k[k];  // 0 = newest
                        state[((uint64_t)c * (RF - 1u) + back) * 64u + t / seq_len] = hc[k];
                    }
                }
            }
        }
    }
}

// Decode: one token per request (t < tokens <= 64); thread = (channel, token).
template <uint32_t RF>
__global__ __launch_bounds__(256) void k44_token_shift_decode_kernel(
    __half *__restrict__ y, const __half *__restrict__ x, const __half *__restrict__ mu,
    __half *__restrict__ state, uint32_t D, uint32_t stride, uint32_t tokens) {
    const uint64_t n = (uint64_t)D * stride;
    for (uint64_t e = (uint64_t)blockIdx.x * 256u + threadIdx.x; e < n;
         e += (uint64_t)gridDim.x * 256u) {
        const uint32_t c = (uint32_t)(e / stride), t = (uint32_t)(e - (uint64_t)c * stride);
        if (t >= tokens) {
            y[e] = __float2half_rn(0.0f);
            continue;
        }
        // The receptive field is a template parameter: every load below is issued at once.
        const __half *m = mu + (uint64_t)c * RF;
        __half *st = state + (uint64_t)c * (RF - 1u) * 64u + t;  // request r = token t
        const __half xe = x[e];
        float mw[RF], prev[RF > 1u ? RF - 1u : 1u];
#pragma unroll
        for (uint32_t i = 0; i < RF; ++i) mw[i] = __half2float(m[i]);
#pragma unroll
        for (uint32_t i = 1; i < RF; ++i) prev[i - 1] = __half2float(st[(i - 1u) * 64u]);
        float acc = mw[0] * __half2float(xe);
#pragma unroll
        for (uint32_t i = 1; i < RF; ++i) acc = fmaf(mw[i], prev[i - 1], acc);
#pragma unroll
        for (uint32_t i = RF - 1u; i > 1u; --i) st[(i - 1u) * 64u] = __float2half_rn(prev[i - 2]);
        if (RF > 1u) st[0] = xe;
        y[e] = f16_of(acc);
    }
}

// Workgroup = 64 tokens x 64 channels: the 64 table rows (128 contiguous bytes each) go through
// LDS and leave as 64 channel rows of 64 tokens (128 contiguous bytes each).
__global__ __launch_bounds__(256) void k44_embed_kernel(__half *__restrict__ y,
                                                        const __half *__restrict__ table,
                                                        const uint32_t *__restrict__ ids,
                                                        uint32_t D, uint32_t vocab,
                                                        uint32_t stride, uint32_t tokens) {
    __shared__ __half tile[64][66];
    const uint32_t t0 = blockIdx.x * 64u, c0 = blockIdx.y * 64u;
    for (uint32_t q = threadIdx.x; q < 64u * 64u; q += 256u) {
        const uint32_t tt = q >> 6, cc = q & 63u;  // read: token tt, channel cc (row-contiguous)
        const uint32_t t = t0 + tt, c = c0 + cc;
        __half v = __float2half_rn(0.0f);
        if (t < tokens && c < D) {
            const uint32_t id = ids[t];
            if (id < vocab) v = table[(uint64_t)id * D + c];
        }
        tile[tt][cc] = v;
    }
    __syncthreads();
    for (uint32_t q = threadIdx.x; q < 64u * 64u; q += 256u) {
        const uint32_t cc = q >> 6, tt = q & 63u;  // write: channel cc, token tt (row-contiguous)
        if (c0 + cc < D) y[(uint64_t)(c0 + cc) * stride + t0 + tt] = tile[tt][cc];
    }
}

// The same gather with 16-byte accesses (D % 8 == 0, 16-byte aligned table and output): a
// thread loads 8 channels of one token's row and stores 8 tokens of one channel, every load
// issued before the first wait (ids and rows clamped into range, invalid ones zeroed after).
// slots (decode, see launch_embed): tokens 0..15 of the workgroup's 64 channels summed
// squared exactly by the 8 threads of each token (threads 0..127), over lanes xor 1, 2, 4.
__global__ __launch_bounds__(256) void k44_embed_vec_kernel(__half *__restrict__ y,
                                                            const __half *__restrict__ table,
                                                            const uint32_t *__restrict__ ids,
                                                            uint32_t D, uint32_t vocab,
                                                            uint32_t stride, uint32_t tokens,
                                                            uint64_t *__restrict__ slots,
                                                            EmbedCopy cp) {
    constexpr uint32_t PITCH = 72u;  // halves per token row: 16-byte rows, spread banks
    __shared__ __attribute__((aligned(16))) __half tile[64 * PITCH];
    const uint32_t t0 = blockIdx.x * 64u, c0 = blockIdx.y * 64u;
    if (cp.rows) {  // the copy carried for a folded token shift (16 bytes per thread and step)
        const uint32_t nth = gridDim.x * gridDim.y * 256u;
        for (uint32_t i = (blockIdx.y * gridDim.x + blockIdx.x) * 256u + threadIdx.x;
             i < 2u * cp.rows; i += nth)
            *reinterpret_cast<uint4 *>(cp.dst + (uint64_t)(i >> 1) * cp.dstride + (i & 1u) * 8u) =
                *reinterpret_cast<const uint4 *>(cp.src + (uint64_t)(i >> 1) * cp.sstride +
                                                 (i & 1u) * 8u);
    }
    uint4 v[2];
    bool ok[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const uint32_t q = threadIdx.x + (uint32_t)r * 256u;
        const uint32_t tt = q >> 3, c = c0 + (q & 7u) * 8u;
        const uint32_t t = t0 + tt;
        const uint32_t id = ids[t < tokens ? t : 0u];
        ok[r] = t < tokens && id < vocab && c < D;
        const uint64_t row = id < vocab ? id : 0u;
        v[r] = *reinterpret_cast<const uint4 *>(table + row * D + (c < D ? c : 0u));
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const uint32_t q = threadIdx.x + (uint32_t)r * 256u;
        *reinterpret_cast<uint4 *>(&tile[(q >> 3) * PITCH + (q & 7u) * 8u]) =
            ok[r] ? v[r] : uint4{0u, 0u, 0u, 0u};
    }
    if (slots && threadIdx.x < 128u) {  // waves 0, 1: tokens 0..15 (uniform per wave)
        const uint4 o = ok[0] ? v[0] : uint4{0u, 0u, 0u, 0u};
        SumSq s = sumsq_zero();
        const uint32_t w4[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
        for (int k = 0; k < 8; ++k) sumsq_add(s, w4[k >> 1] >> (16 * (k & 1)));
        s = sumsq_norm(s);
#pragma unroll
        for (int m = 1; m < 8; m <<= 1) {
            SumSq x;
            x.l0 = (uint32_t)__shfl_xor((int)(uint32_t)s.l0, m, 64);
            x.l1 = (uint32_t)__shfl_xor((int)(uint32_t)s.l1, m, 64);
            x.l2 = (uint32_t)__shfl_xor((int)(uint32_t)s.l2, m, 64);
            x.sp = (uint32_t)__shfl_xor((int)s.sp, m, 64);
            sumsq_merge(s, x);
            s = sumsq_norm(s);
        }
        if ((threadIdx.x & 7u) == 0u) {
            uint64_t *sl = slots + ((uint64_t)blockIdx.y * 16u + (threadIdx.x >> 3)) * 2u;
            sl[0] = s.l0 | (s.l1 << 32);
            sl[1] = (uint64_t)(uint32_t)s.l2 | ((uint64_t)s.sp << 32);
        }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const uint32_t q = threadIdx.x + (uint32_t)r * 256u;
        const uint32_t cc = q >> 3, tg = (q & 7u) * 8u;  // channel c0 + cc, tokens tg .. tg + 7
        if (c0 + cc >= D) continue;
        uint4 o;
        __half *oh = reinterpret_cast<__half *>(&o);
#pragma unroll
        for (uint32_t j = 0; j < 8u; ++j) oh[j] = tile[(tg + j) * PITCH + cc];
        *reinterpret_cast<uint4 *>(y + (uint64_t)(c0 + cc) * stride + t0 + tg) = o;
    }
}

// ARGMAX pass 1: workgroup = 64 tokens x one chunk of channels; lane (16 per channel row) owns
// 4 tokens, the 16 row groups of the workgroup stride the chunk.  Ties keep the lowest channel
// (channels are visited in ascending order per thread, and merged lowest-index-first).
__device__ __forceinline__ void amax_merge(float &bv, uint32_t &bi, float v, uint32_t i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

__global__ __launch_bounds__(256) void k44_argmax_partial_kernel(
    float *__restrict__ pval, uint32_t *__restrict__ pidx, const __half *__restrict__ x,
    uint32_t V, uint32_t stride, uint32_t chunk) {
    __shared__ float sv[16][64];
    __shared__ uint32_t si[16][64];
    const uint32_t grp = threadIdx.x >> 4, q = threadIdx.x & 15u;
    const uint32_t t0 = blockIdx.x * 64u + q * 4u;
    const uint32_t c_begin = blockIdx.y * chunk, c_end = min(V, c_begin + chunk);
    float bv[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    uint32_t bi[4] = {0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu};
    // 8 channel rows per thread in flight (the merge rule is order-independent).
    constexpr uint32_t UNR = 8;
    uint32_t c = c_begin + grp;
    for (; c + (UNR - 1u) * 16u < c_end; c += UNR * 16u) {
        gd_u2 v[UNR];
#pragma unroll
        for (uint32_t u = 0; u < UNR; ++u)
            v[u] = *reinterpret_cast<const gd_u2 *>(x + (uint64_t)(c + u * 16u) * stride + t0);
#pragma unroll
        for (uint32_t u = 0; u < UNR; ++u) {
            const __half *h = reinterpret_cast<const __half *>(&v[u]);
#pragma unroll
            for (int k = 0; k < 4; ++k) amax_merge(bv[k], bi[k], __half2float(h[k]), c + u * 16u);
        }
    }
    for (; c < c_end; c += 16u) {
        const gd_u2 v = *reinterpret_cast<const gd_u2 *>(x + (uint64_t)c * stride + t0);
        const __half *h = reinterpret_cast<const __half *>(&v);
#pragma unroll
        for (int k = 0; k < 4; ++k) amax_merge(bv[k], bi[k], __half2float(h[k]), c);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        sv[grp][q * 4u + k] = bv[k];
        si[grp][q * 4u + k] = bi[k];
    }
    __syncthreads();
    if (threadIdx.x < 64u) {
        float v = sv[0][threadIdx.x];
        uint32_t i = si[0][threadIdx.x];
        for (int g2 = 1; g2 < 16; ++g2) amax_merge(v, i, sv[g2][threadIdx.x], si[g2][threadIdx.x]);
        const uint64_t o = (uint64_t)blockIdx.y * (gridDim.x * 64u) + blockIdx.x * 64u + threadIdx.x;
        pval[o] = v;
        pidx[o] = i;
    }
}

// Pass 1 with 16-byte loads (16-byte aligned logits): 8 lanes per 64-token row, each owning 8
// tokens; the 32 row groups of the workgroup stride the chunk, UNR rows in flight per thread.
// Measured on the config-5 prefill logits (32,000 x 8,192, 512 workgroups): 4 rows in flight
// 85 us, 8 rows 102 us, 16 rows 115 us; a decode chunk (8 rows per thread) takes 8 (one round
// trip).
template <uint32_t UNR>
__global__ __launch_bounds__(256) void k44_argmax_partial16_kernel(
    float *__restrict__ pval, uint32_t *__restrict__ pidx, const __half *__restrict__ x,
    uint32_t V, uint32_t stride, uint32_t chunk) {
    __shared__ float sv[32][64];
    __shared__ uint32_t si[32][64];
    const uint32_t grp = threadIdx.x >> 3, q = threadIdx.x & 7u;
    const uint32_t t0 = blockIdx.x * 64u + q * 8u;
    const uint32_t c_begin = blockIdx.y * chunk, c_end = min(V, c_begin + chunk);
    float bv[8];
    uint32_t bi[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        bv[k] = -INFINITY;
        bi[k] = 0xffffffffu;
    }
    uint32_t c = c_begin + grp;
    for (; c + (UNR - 1u) * 32u < c_end; c += UNR * 32u) {
        uint4 v[UNR];
#pragma unroll
        for (uint32_t u = 0; u < UNR; ++u)
            v[u] = *reinterpret_cast<const uint4 *>(x + (uint64_t)(c + u * 32u) * stride + t0);
#pragma unroll
        for (uint32_t u = 0; u < UNR; ++u) {
            const __half *h = reinterpret_cast<const __half *>(&v[u]);
#pragma unroll
            for (int k = 0; k < 8; ++k) amax_merge(bv[k], bi[k], __half2float(h[k]), c + u * 32u);
        }
    }
    for (; c < c_end; c += 32u) {
        const uint4 v = *reinterpret_cast<const uint4 *>(x + (uint64_t)c * stride + t0);
        const __half *h = reinterpret_cast<const __half *>(&v);
#pragma unroll
        for (int k = 0; k < 8; ++k) amax_merge(bv[k], bi[k], __half2float(h[k]), c);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        sv[grp][q * 8u + k] = bv[k];
        si[grp][q * 8u + k] = bi[k];
    }
    __syncthreads();
    if (threadIdx.x < 64u) {
        float v = sv[0][threadIdx.x];
        uint32_t i = si[0][threadIdx.x];
        for (int g2 = 1; g2 < 32; ++g2) amax_merge(v, i, sv[g2][threadIdx.x], si[g2][threadIdx.x]);
        const uint64_t o = (uint64_t)blockIdx.y * (gridDim.x * 64u) + blockIdx.x * 64u + threadIdx.x;
        pval[o] = v;
        pidx[o] = i;
    }
}

// ARGMAX pass 2: one wave per token; lanes take chunks lane, lane + 64, ... and the wave merges
// them with the same rule (higher value, then lower channel), which is order-independent.
__global__ __launch_bounds__(64) void k44_argmax_final_kernel(
    uint32_t *__restrict__ ids, uint32_t *__restrict__ history,
    const uint32_t *__restrict__ step_ctr, uint32_t hist_steps, uint32_t tokens,
    const float *__restrict__ pval, const uint32_t *__restrict__ pidx, uint32_t chunks,
    uint32_t ld) {
    const uint32_t t = blockIdx.x, lane = threadIdx.x;
    float v = -INFINITY;
    uint32_t i = 0xffffffffu;
    for (uint32_t k = lane; k < chunks; k += 64u)
        amax_merge(v, i, pval[(uint64_t)k * ld + t], pidx[(uint64_t)k * ld + t]);
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const float ov = __shfl_xor(v, m, 64);
        const uint32_t oi = __shfl_xor(i, m, 64);
        amax_merge(v, i, ov, oi);
    }
    if (lane == 0u) {
        const uint32_t id = i == 0xffffffffu ? 0u : i;
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
                          uint32_t stride, uint32_t tokens, float eps, hipStream_t stream,
                          const RmsShift *shift, const uint64_t *slots, uint32_t n_slots) {
    if (stride % 64u != 0u || D == 0u || tokens == 0u || tokens > stride)
        return hipErrorInvalidValue;
    // producers' slots: the decode octet kernel only (16 tokens per slot; its exact sums are
    // what they replace)
    if (slots && ((shift && shift->seq_len) || tokens > 16u || n_slots == 0u))
        return hipErrorInvalidValue;
    // token columns >= tokens are not written; octets per workgroup: the widest that still
    // gives >= 256 workgroups (coalesced rows), else 1 octet and channel slices
    const uint32_t octets = (tokens + 7u) / 8u;
    uint32_t oct = 8u;
    while (oct > 1u && (octets + oct - 1u) / oct < 256u) oct >>= 1;
    uint32_t chunks = (octets + oct - 1u) / oct;
    uint32_t slices = (256u + chunks - 1u) / chunks;
    const uint32_t max_slices = (D + 255u) / 256u;
    slices = slices < max_slices ? slices : max_slices;
    const uint32_t cslice = (D + slices - 1u) / slices;
    RmsShift sh{};
    if (shift && shift->seq_len) {
        // Fused prefill token shift: the register-resident wide kernel with the shift.
        if (!rmsnorm_shift_prefill_ok(D, stride, tokens, shift->rf, shift->seq_len))
            return hipErrorInvalidValue;
        const dim3 gw(tokens / 32u);
#define K44_RMSP(C, R)                                                                          \
    hipLaunchKernelGGL((k44_rmsnorm_shift_prefill_kernel<C, R>), gw, dim3(1024), 0, stream, y, x, \
                       gamma, D, stride, eps, shift->y2, shift->mu, shift->state, shift->seq_len)
#define K44_RMSP_RF(C)                  \
    switch (shift->rf) {                \
    case 1u: K44_RMSP(C, 1u); break;    \
    case 2u: K44_RMSP(C, 2u); break;    \
    case 3u: K44_RMSP(C, 3u); break;    \
    case 4u: K44_RMSP(C, 4u); break;    \
    default: K44_RMSP(C, 5u); break;    \
    }
        if (D <= 1024u) {
            K44_RMSP_RF(4)
        } else {
            K44_RMSP_RF(8)
        }
#undef K44_RMSP_RF
#undef K44_RMSP
        return hipGetLastError();
    }
    if (shift) {
        // Fused decode token shift: one channel per thread, every octet of the stride.
        if (oct != 1u || cslice > 256u || tokens > 64u || stride != 64u || shift->rf == 0u ||
            shift->rf > 9u || (shift->rf > 1u && !shift->state))
            return hipErrorInvalidValue;
        sh = *shift;
        sh.tokens = tokens;
        chunks = stride / 8u;
    }
    // Prefill-sized token counts without a fused shift: the register-resident wide kernel
    // (32 tokens x all channels per workgroup) when the channels fit 16 per thread.
    if (!shift && !slots && tokens % 32u == 0u && tokens / 32u >= 256u && D <= 16u * 256u) {
        const dim3 gw(tokens / 32u);
#define K44_RMSW(C)                                                                            \
    hipLaunchKernelGGL((k44_rmsnorm_regs_kernel<C>), gw, dim3(1024), 0, stream, y, x, gamma, D, \
                       stride, eps)
        const uint32_t cpt = (D + 255u) / 256u;
        if (cpt <= 4u) {
            K44_RMSW(4);
        } else if (cpt <= 8u) {
            K44_RMSW(8);
        } else {
            K44_RMSW(16);
        }
#undef K44_RMSW
        return hipGetLastError();
    }
    const dim3 grid(chunks, (D + cslice - 1u) / cslice);
#define K44_RMS(O, R) \
    hipLaunchKernelGGL((k44_rmsnorm_kernel<O, R>), grid, dim3(256), 0, stream, y, x, gamma, D, stride, eps, cslice, sh, slots, n_slots)
    if (shift) {
        switch (sh.rf) {
        case 1u: K44_RMS(1, 1u); break;
        case 2u: K44_RMS(1, 2u); break;
        case 3u: K44_RMS(1, 3u); break;
        case 4u: K44_RMS(1, 4u); break;
        case 5u: K44_RMS(1, 5u); break;
        case 6u: K44_RMS(1, 6u); break;
        case 7u: K44_RMS(1, 7u); break;
        case 8u: K44_RMS(1, 8u); break;
        default: K44_RMS(1, 9u); break;
        }
    } else {
        switch (oct) {
        case 8u: K44_RMS(8, 0u); break;
        case 4u: K44_RMS(4, 0u); break;
        case 2u: K44_RMS(2, 0u); break;
        default: K44_RMS(1, 0u); break;
        }
    }
#undef K44_RMS
    return hipGetLastError();
}

hipError_t launch_mul(__half *y, const __half *a, const __half *b, uint64_t n,
                      hipStream_t stream) {
    if (n % 8u != 0u) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k44_mul_kernel, dim3(grid_for(n / 8u)), dim3(256), 0, stream, y, a, b,
                       n / 8u);
    return hipGetLastError();
}

hipError_t launch_mul3(__half *y, const __half *a, const __half *b, const __half *c, uint64_t n,
                       hipStream_t stream) {
    if (n % 8u != 0u) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k44_mul3_kernel, dim3(grid_for(n / 8u)), dim3(256), 0, stream, y, a, b, c,
                       n / 8u);
    return hipGetLastError();
}

hipError_t launch_token_shift(__half *y, const __half *x, const __half *mu, __half *state,
                              uint32_t D, uint32_t stride, uint32_t tokens, uint32_t rf,
                              uint32_t seq_len, int decode, hipStream_t stream) {
    if (rf == 0u || rf > 9u || seq_len == 0u || stride % 64u != 0u ||
        (decode && ((rf > 1u && !state) || tokens > 64u)))
        return hipErrorInvalidValue;
    if (decode) {
        const dim3 grid(grid_for((uint64_t)D * stride));
        switch (rf) {
#define K44_TSD(R)                                                                           \
    case R:                                                                                  \
        hipLaunchKernelGGL(k44_token_shift_decode_kernel<R>, grid, dim3(256), 0, stream, y, x, \
                           mu, state, D, stride, tokens);                                    \
        break;
            K44_TSD(1) K44_TSD(2) K44_TSD(3) K44_TSD(4) K44_TSD(5) K44_TSD(6) K44_TSD(7)
            K44_TSD(8) K44_TSD(9)
#undef K44_TSD
        default: return hipErrorInvalidValue;
        }
    } else {
        const uint32_t chunks = stride / 8u;
        const uint32_t gx = (chunks + 255u) / 256u;
        const uint32_t groups = (D + TS_CPC - 1u) / TS_CPC;
        const uint32_t gy = groups < 65535u ? groups : 65535u;
        switch (rf) {
#define K44_TSP(R)                                                                             \
    case R:                                                                                    \
        hipLaunchKernelGGL(k44_token_shift_prefill_kernel<R>, dim3(gx, gy), dim3(256), 0,      \
                           stream, y, x, mu, state, D, stride, tokens, seq_len);               \
        break;
            K44_TSP(1) K44_TSP(2) K44_TSP(3) K44_TSP(4) K44_TSP(5) K44_TSP(6) K44_TSP(7)
            K44_TSP(8) K44_TSP(9)
#undef K44_TSP
        default: return hipErrorInvalidValue;
        }
    }
    return hipGetLastError();
}

hipError_t launch_embed(__half *y, const __half *table, const uint32_t *ids, uint32_t D,
                        uint32_t vocab, uint32_t stride, uint32_t tokens, hipStream_t stream,
                        uint64_t *slots, const EmbedCopy &cp) {
    if (stride % 64u != 0u || D == 0u) return hipErrorInvalidValue;
    // the carried copy: 16-byte aligned rows of 16 halves, with the slot form only
    if (cp.rows && (!slots || reinterpret_cast<uintptr_t>(cp.src) % 16u != 0u ||
                    reinterpret_cast<uintptr_t>(cp.dst) % 16u != 0u || cp.sstride % 8u != 0u ||
                    cp.dstride % 8u != 0u))
        return hipErrorInvalidValue;
    const dim3 grid(stride / 64u, (D + 63u) / 64u);
    const bool vec = tokens > 0u && D % 8u == 0u && reinterpret_cast<uintptr_t>(table) % 16u == 0u &&
                     reinterpret_cast<uintptr_t>(y) % 16u == 0u;
    // slots: the vector kernel over one 64-token block with at most 16 tokens
    if (slots && (!vec || stride != 64u || tokens > 16u || D % 64u != 0u))
        return hipErrorInvalidValue;
    if (vec)
        hipLaunchKernelGGL(k44_embed_vec_kernel, grid, dim3(256), 0, stream, y, table, ids, D,
                           vocab, stride, tokens, slots, cp);
    else
        hipLaunchKernelGGL(k44_embed_kernel, grid, dim3(256), 0, stream, y, table, ids, D, vocab,
                           stride, tokens);
    return hipGetLastError();
}

__global__ void k44_step_inc_kernel(uint32_t *ctr) { *ctr += 1u; }

// dst[r * cols + c] = src[r * row_stride + c]: `cols` elements of `rows` strided rows, packed
// (one contiguous copy to the host afterwards instead of a row-by-row 2-D transfer).
__global__ __launch_bounds__(256) void k44_gather_cols_kernel(uint16_t *__restrict__ dst,
                                                              const uint16_t *__restrict__ src,
                                                              uint64_t rows, uint64_t row_stride,
                                                              uint64_t cols) {
    const uint64_t n = rows * cols;
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * 256u) {
        const uint64_t r = i / cols, c = i - r * cols;
        dst[i] = src[r * row_stride + c];
    }
}

hipError_t launch_gather_cols(uint16_t *dst, const uint16_t *src, uint64_t rows,
                              uint64_t row_stride, uint64_t cols, hipStream_t stream) {
    hipLaunchKernelGGL(k44_gather_cols_kernel, dim3(grid_for(rows * cols)), dim3(256), 0, stream,
                       dst, src, rows, row_stride, cols);
    return hipGetLastError();
}

static uint32_t argmax_chunk_len(uint32_t V, uint32_t stride) {
    const uint32_t tiles = stride / 64u;
    uint32_t chunks = (512u + tiles - 1u) / tiles;  // ~512 workgroups in pass 1
    const uint32_t max_chunks = (V + 255u) / 256u;  // >= 256 channels per chunk
    chunks = chunks < max_chunks ? chunks : max_chunks;
    chunks = chunks ? chunks : 1u;
    return (V + chunks - 1u) / chunks;
}

size_t argmax_scratch_floats(uint32_t V, uint32_t stride) {
    const uint32_t chunk = argmax_chunk_len(V, stride);
    return 2u * (size_t)((V + chunk - 1u) / chunk) * stride;
}

hipError_t launch_argmax(uint32_t *ids, uint32_t *history, uint32_t *step_ctr,
                         uint32_t hist_steps, const __half *x, uint32_t V, uint32_t stride,
                         uint32_t tokens, float *scratch, hipStream_t stream) {
    if (stride % 64u != 0u || V == 0u || !scratch) return hipErrorInvalidValue;
    const uint32_t chunk = argmax_chunk_len(V, stride);
    const uint32_t used = (V + chunk - 1u) / chunk;
    float *pval = scratch;
    uint32_t *pidx = reinterpret_cast<uint32_t *>(scratch + (uint64_t)used * stride);
    if (reinterpret_cast<uintptr_t>(x) % 16u == 0u && chunk <= 8u * 32u)
        hipLaunchKernelGGL(k44_argmax_partial16_kernel<8>, dim3(stride / 64u, used), dim3(256), 0,
                           stream, pval, pidx, x, V, stride, chunk);
    else if (reinterpret_cast<uintptr_t>(x) % 16u == 0u)
        hipLaunchKernelGGL(k44_argmax_partial16_kernel<4>, dim3(stride / 64u, used), dim3(256), 0,
                           stream, pval, pidx, x, V, stride, chunk);
    else
        hipLaunchKernelGGL(k44_argmax_partial_kernel, dim3(stride / 64u, used), dim3(256), 0,
                           stream, pval, pidx, x, V, stride, chunk);
    hipLaunchKernelGGL(k44_argmax_final_kernel, dim3(tokens), dim3(64), 0, stream, ids, history,
                       step_ctr, hist_steps, tokens, pval, pidx, used, stride);
    if (history) hipLaunchKernelGGL(k44_step_inc_kernel, dim3(1), dim3(1), 0, stream, step_ctr);
    return hipGetLastError();
}

}  // namespace k44dev
