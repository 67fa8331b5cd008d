// k44_sumsq.hpp — RMSNorm arithmetic: exact sums of squares of fp16 values (decode-sized
// plans) and the normalised element expression.
//
// RMSNorm (reference kernels/common/kernel44_valu_pack.cuh:104-134) needs, per token, the sum
// of x^2 over the channels.  Summed in fp32, the result depends on the order of the additions,
// so a norm computed by one kernel and the same norm assembled from the partial sums of the
// workgroups that produced its input (in another order) would differ in the last bits.  Here
// the sum is exact: an fp16 value is mm * 2^(e - 25) (mm = the 11-bit significand, e = the
// exponent field, subnormals with e = 1), so x^2 = mm^2 * 2^(2e - 50) is the 22-bit integer
// mm^2 shifted left by 2e - 2 (0..58) in units of 2^-48.  Squares are added into three 32-bit
// limbs held in 64-bit accumulators (no carries while adding: up to 2^32 terms per limb), so
// any grouping of the terms gives the same integer.  The integer is rounded to fp32 once (round
// to nearest even), and inf / NaN inputs give an inf / NaN sum, as an fp32 sum would.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace k44dev {

// fp16 of an fp32 value, rounded to fp32 first as written: the opaque register move keeps the
// compiler from fusing the multiply or FMA that produced `v` and the conversion into one
// mixed-precision FMA (a single rounding) — which it may do at one use of an expression and
// not at another (a normalised value stored and the same value recomputed for the fused token
// shift, or a fused and a stand-alone token shift, differed in the last bit).
__device__ __forceinline__ __half f16_of(float v) {
    asm volatile("" : "+v"(v));
    return __float2half_rn(v);
}

// RMSNorm output fp16(x * inv * gamma), both products in fp32 (the norm kernels and the
// gathers of waves that apply a folded norm use this one expression).
__device__ __forceinline__ __half norm_scale(__half x, float inv, float g) {
    return f16_of(__half2float(x) * inv * g);
}

struct SumSq {
    uint64_t l0, l1, l2;  // limbs: value = l0 + l1 * 2^32 + l2 * 2^64 (units of 2^-48)
    uint32_t sp;          // bit 0: an infinite input, bit 1: a NaN input
};

__host__ __device__ __forceinline__ SumSq sumsq_zero() { return SumSq{0u, 0u, 0u, 0u}; }

// s += x^2 for the fp16 value with bits h (low 16 bits of h).
__host__ __device__ __forceinline__ void sumsq_add(SumSq &s, uint32_t h) {
    const uint32_t e = (h >> 10) & 31u, m = h & 1023u;
    const uint32_t mm = e ? (m | 1024u) : m;
    const uint32_t sh = e > 1u ? 2u * e - 2u : 0u;  // e = 31 (inf / NaN) is flagged below
    const uint64_t v = (uint64_t)(mm * mm);          // < 2^22
    const bool up = sh >= 32u;
    const uint64_t w = v << (up ? sh - 32u : sh);    // < 2^54
    const uint64_t lo = w & 0xffffffffull, hi = w >> 32;
    s.l0 += up ? 0ull : lo;
    s.l1 += up ? lo : hi;
    s.l2 += up ? hi : 0ull;
    s.sp |= e == 31u ? (m ? 2u : 1u) : 0u;
}

__host__ __device__ __forceinline__ void sumsq_merge(SumSq &s, const SumSq &o) {
    s.l0 += o.l0;
    s.l1 += o.l1;
    s.l2 += o.l2;
    s.sp |= o.sp;
}

// Carries propagated: every limb below 2^32 except the top one (same value).
__host__ __device__ __forceinline__ SumSq sumsq_norm(SumSq s) {
    s.l1 += s.l0 >> 32;
    s.l0 &= 0xffffffffull;
    s.l2 += s.l1 >> 32;
    s.l1 &= 0xffffffffull;
    return s;
}

// The exact sum rounded to fp32 (round to nearest even).  The 128-bit integer H:L is brought to
// 64 bits with the bits shifted out ORed into the lowest one (rounding to odd at 64 bits), and
// that integer is converted with one rounding: rounding to odd at >= 26 bits and then to
// nearest even at 24 gives the nearest-even rounding of the exact value.
__host__ __device__ __forceinline__ float sumsq_value(SumSq s) {
    if (s.sp) return (s.sp & 2u) ? __builtin_nanf("") : __builtin_inff();
    s = sumsq_norm(s);
    const uint64_t L = s.l0 | (s.l1 << 32), H = s.l2;
    if (H == 0ull) return __builtin_ldexpf((float)L, -48);
    const int k = 64 - __builtin_clzll(H);  // bits of H (1..64)
    uint64_t T = (L >> k) | (k < 64 ? (H << (64 - k)) : 0ull);
    if (k == 64) T = H;
    const uint64_t dropped = k < 64 ? (L & ((1ull << k) - 1ull)) : L;
    T |= dropped != 0ull ? 1ull : 0ull;
    return __builtin_ldexpf((float)T, k - 48);
}

// RMSNorm scale of a token from its exact sum of squares over D channels.
__device__ __forceinline__ float rms_inv(const SumSq &s, uint32_t D, float eps) {
    return rsqrtf(sumsq_value(s) / (float)D + eps);
}

// 64-lane wave reduction of a SumSq over the lanes that share (lane & (span - 1)), i.e. xor
// distances span, 2 span, ... 32 (span a power of two).  Exact, so the order does not matter.
__device__ __forceinline__ SumSq sumsq_wave_reduce(SumSq s, int span) {
    s = sumsq_norm(s);  // every limb < 2^32 except l2 (small): 32-bit shuffles of each
    for (int m = span; m < 64; m <<= 1) {
        SumSq o;
        o.l0 = (uint32_t)__shfl_xor((int)(uint32_t)s.l0, m, 64);
        o.l1 = (uint32_t)__shfl_xor((int)(uint32_t)s.l1, m, 64);
        o.l2 = (uint32_t)__shfl_xor((int)(uint32_t)s.l2, m, 64);
        o.sp = (uint32_t)__shfl_xor((int)s.sp, m, 64);
        sumsq_merge(s, o);
        s = sumsq_norm(s);
    }
    return s;
}

// Per-token RMSNorm scales of TK tokens (t0 .. t0 + TK - 1) from the exact sums of squares
// that the n producer tiles of the norm's input stored, one slot of 16 tokens x 2 words per
// tile (limbs 0 | 1 << 32, limb 2 | flags << 32).  Called by the whole 256-thread workgroup:
// thread (token tid % TK, part tid / TK) adds slots part, part + 256 / TK, ... (exact: any
// order gives the same integer), the parts of a token meet by shuffles within the wave and
// across the 4 waves in LDS; inv[k] holds token t0 + k's scale after the call's last barrier.
// In two steps, so that a kernel can issue the slot loads before its other loads and add them
// once they have arrived: rms_slots_issue loads the thread's first 4 slots (up to 4 x 256 / TK
// slots in all), rms_slots_finish adds them (and loads any further slots itself).
template <uint32_t TK>
struct SlotLoads {
    uint64_t lo[4], hi[4];
};

template <uint32_t TK>
__device__ __forceinline__ void rms_slots_issue(const uint64_t *slots, uint32_t n, uint32_t t0,
                                                SlotLoads<TK> &p) {
    static_assert(TK == 8u || TK == 16u, "tokens per pass");
    constexpr uint32_t PARTS = 256u / TK;
    typedef const __attribute__((address_space(1))) uint64_t gu64c;
    const uint32_t tk = threadIdx.x % TK, pt = threadIdx.x / TK;
#pragma unroll
    for (uint32_t u = 0; u < 4u; ++u) {
        const uint32_t i = min(pt + PARTS * u, n - 1u);
        const gu64c *w = (const gu64c *)slots + ((uint64_t)i * 16u + t0 + tk) * 2u;
        p.lo[u] = w[0];
        p.hi[u] = w[1];
    }
}

template <uint32_t TK>
__device__ __forceinline__ void rms_slots_finish(const SlotLoads<TK> &p, const uint64_t *slots,
                                                 uint32_t n, uint32_t t0, uint32_t D, float eps,
                                                 uint4 (&part)[4][TK], float (&inv)[TK]) {
    constexpr uint32_t PARTS = 256u / TK;
    typedef const __attribute__((address_space(1))) uint64_t gu64c;
    const uint32_t tk = threadIdx.x % TK, pt = threadIdx.x / TK;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    SumSq q = sumsq_zero();
    auto add4 = [&](uint32_t i0, const uint64_t (&lo)[4], const uint64_t (&hi)[4]) {
#pragma unroll
        for (uint32_t u = 0; u < 4u; ++u)
            if (i0 + PARTS * u < n) {
                q.l0 += lo[u] & 0xffffffffull;
                q.l1 += lo[u] >> 32;
                q.l2 += hi[u] & 0xffffffffull;
                q.sp |= (uint32_t)(hi[u] >> 32);
            }
    };
    add4(pt, p.lo, p.hi);
    for (uint32_t i0 = pt + 4u * PARTS; i0 < n; i0 += 4u * PARTS) {
        uint64_t lo[4], hi[4];
#pragma unroll
        for (uint32_t u = 0; u < 4u; ++u) {
            const uint32_t i = min(i0 + PARTS * u, n - 1u);
            const gu64c *w = (const gu64c *)slots + ((uint64_t)i * 16u + t0 + tk) * 2u;
            lo[u] = w[0];
            hi[u] = w[1];
        }
        add4(i0, lo, hi);
    }
    q = sumsq_wave_reduce(q, (int)TK);  // the lanes of one token in this wave
    if (lane < TK) part[wave][lane] = uint4{(uint32_t)q.l0, (uint32_t)q.l1, (uint32_t)q.l2, q.sp};
    __syncthreads();
    if (threadIdx.x < TK) {
        SumSq t = sumsq_zero();
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint4 x = part[v][threadIdx.x];
            t.l0 += x.x;
            t.l1 += x.y;
            t.l2 += x.z;
            t.sp |= x.w;
        }
        inv[threadIdx.x] = rms_inv(t, D, eps);
    }
    __syncthreads();
}

template <uint32_t TK>
__device__ __forceinline__ void rms_inv_from_slots(const uint64_t *slots, uint32_t n,
                                                   uint32_t t0, uint32_t D, float eps,
                                                   uint4 (&part)[4][TK], float (&inv)[TK]) {
    SlotLoads<TK> p;
    rms_slots_issue<TK>(slots, n, t0, p);
    rms_slots_finish<TK>(p, slots, n, t0, D, eps, part, inv);
}

}  // namespace k44dev
