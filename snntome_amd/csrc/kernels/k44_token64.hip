// k44_token64.hip — the stand-alone Token64 wave and the GPU form of the WMMA weight interleave.
//
// Token64 wave (semantics of the reference's whitepaper launcher, whitepaper/sparse_wmma_kernel/
// kernels/kernel44_immutable.cuh:200-297): activations in 64-token tiles,
//     X[tile][Cin][64], Y[tile][Cout][64] fp16,
// clusters of `cluster` (a multiple of 16) consecutive neurons share one index row of
// B = 16*B_vec16 input positions idx[c][k] (any positions, 64-bit addressing throughout), weights in
// the RDNA4 WMMA vector order (k44_plan_types.hpp convert_raw_to_wmma), bias always added,
//     Y[t][j][m] = fp16_round_toward_zero(bias[j] + sum_k W[j][k] * X[t][idx[j/cluster][k]][m]).
//
// MI355X mapping.  One wave = one 64-token tile x 16*NB neurons of one cluster (NB = 4, 2, 1:
// the widest that divides the cluster); a workgroup holds 4 waves on 4 consecutive tiles (same
// neurons, so the A fragments are shared through L1).  Per 32-deep k-step the wave gathers its
// 32 index rows (128 bytes each, 8 lanes x 16 bytes per row) into a private LDS tile, and the B
// operand of v_mfma_f32_16x16x32_f16 comes out with ds_read_b64_tr_b16 (8 positions of one
// token per lane), exactly as in the dense-cluster tile kernel.  A fragments are read straight
// from the WMMA-ordered weights: MFMA lane l needs row 16*nb + (l & 15), columns 32*ks + 8*(l>>4)
// .. +8, which is WMMA vector ((nb * B_vec16 + 2*ks + (l >> 5)) * 32 + (l & 31)).  The next
// k-step's rows and fragments are loaded while the current one is multiplied; the index words
// are loaded two k-steps ahead.  An odd B_vec16 leaves the last k-step half empty: those rows
// and fragments are zero.  An index word >= Cin reads as a zero row (the reference would read
// outside X).
#include <cstdlib>

#include "k44_launch.hpp"
#include "k44_mfma_dma.hpp"

namespace k44dev {

template <int NB>
__global__ __launch_bounds__(256) void k44_token64_kernel(Token64Args a) {
    constexpr int PITCH = 72;  // halves per LDS row: 64 tokens + 16-byte skew
    __shared__ __attribute__((aligned(16))) _Float16 xs[4][32][PITCH];
    const int lane = (int)(threadIdx.x & 63u), wave = (int)(threadIdx.x >> 6);
    const uint32_t tile = blockIdx.y * 4u + (uint32_t)wave;
    if (tile >= a.tiles) return;  // no workgroup barrier in this kernel
    const uint32_t j0 = blockIdx.x * 16u * NB;
    const uint32_t B = a.B_vec16 * 16u;
    const uint32_t ksteps = (a.B_vec16 + 1u) / 2u;
    const uint32_t *irow = a.idx + (uint64_t)(j0 / a.cluster) * B;
    const __half *xt = a.X + (uint64_t)tile * a.Cin * 64u;
    const int gr = lane >> 3, gc = (lane & 7) * 8;  // gather: row gr (+8i), tokens gc..gc+7
    const uint4 *wrow = a.w_wmma + (uint64_t)(j0 / 16u) * a.B_vec16 * 32u + (lane & 31);
    const int g = lane >> 4;

    f4_t acc[NB][4];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        f4_t b0 = {0.0f, 0.0f, 0.0f, 0.0f};
        if (a.bias) {
#pragma unroll
            for (int i = 0; i < 4; ++i) b0[i] = __half2float(a.bias[j0 + 16u * nb + 4u * g + i]);
        }
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) acc[nb][tb] = b0;
    }

    auto load_idx = [&](uint32_t ks, uint32_t (&ix)[4]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t k = 32u * ks + 8u * i + (uint32_t)gr;
            const uint32_t v = k < B ? irow[k] : 0xffffffffu;
            ix[i] = v < a.Cin ? v : 0xffffffffu;  // out-of-range positions read as zero rows
        }
    };
    auto load_x = [&](const uint32_t (&ix)[4], u4_t (&x)[4]) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            x[i] = ix[i] != 0xffffffffu
                       ? *reinterpret_cast<const u4_t *>(xt + (uint64_t)ix[i] * 64u + gc)
                       : u4_t{0u, 0u, 0u, 0u};
    };
    auto load_a = [&](uint32_t ks, h8_t (&af)[NB]) {
        const uint32_t kb = 2u * ks + (uint32_t)(lane >> 5);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
            af[nb] = kb < a.B_vec16
                         ? __builtin_bit_cast(h8_t, wrow[((uint64_t)nb * a.B_vec16 + kb) * 32u])
                         : h8_t{};
    };

    uint32_t ia[4], ib[4];
    u4_t xr[4];
    h8_t ar[NB];
    load_idx(0u, ia);
    load_idx(min(1u, ksteps - 1u), ib);
    load_x(ia, xr);
    load_a(0u, ar);
    const int tr_row = 8 * g + ((lane & 15) >> 2), tr_col = 4 * (lane & 3);
    for (uint32_t ks = 0; ks < ksteps; ++ks) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<u4_t *>(&xs[wave][8 * i + gr][gc]) = xr[i];
        h8_t af[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) af[nb] = ar[nb];
        // Next k-step in flight (clamped at the end: a re-read of the last step, unused).
        const uint32_t kn = min(ks + 1u, ksteps - 1u);
#pragma unroll
        for (int i = 0; i < 4; ++i) ia[i] = ib[i];
        load_idx(min(ks + 2u, ksteps - 1u), ib);
        load_x(ia, xr);
        load_a(kn, ar);
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            const _Float16 *p = &xs[wave][tr_row][tr_col + 16 * tb];
            const h4_t lo = lds_read_tr16(p);
            const h4_t hi = lds_read_tr16(p + 4 * PITCH);
            const h8_t b = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                acc[nb][tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[nb], b, acc[nb][tb], 0, 0, 0);
        }
    }

    // C layout: lane holds C[4g + i][lane & 15] of every 16x16 tile; round toward zero.
    __half *yt = a.Y + ((uint64_t)tile * a.Cout + j0) * 64u + (lane & 15);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int tb = 0; tb < 4; ++tb)
                yt[(uint64_t)(16 * nb + 4 * g + i) * 64u + 16u * tb] = __float2half_rz(acc[nb][tb][i]);
}

// ---------------------------------------------------------------------------------------------
// LDS-ring kernel for the large shapes: clusters of a multiple of 64 neurons, batches of whole
// groups of TW tiles, even B_vec16 (whole 32-deep k-steps), B <= 4096.  Workgroup = 64*NBK
// neurons of one cluster x TW tiles.  The cluster's index row is staged in LDS once; then every
// k-step's 32 gathered rows per tile (128 B each: one global_load_lds_dwordx4 covers 8 rows) and
// its A fragments (1 KiB per 16-neuron block, contiguous in the WMMA order) go memory -> LDS
// directly, into a ring of NBUF stages with NBUF-1 in flight, synchronised as the dense-cluster
// LDS-ring kernel (lds_ring, k44_mfma_dma.hpp): per stage a vmcnt wait + bare s_barrier, LDS reads
// in inline asm with an explicit lgkmcnt wait.  Rows of out-of-range indices are read from a
// zero row in device memory.
//
// Producer and consumer waves.  NBK*TW consumer waves each own one 64-neuron x 64-token output
// block and only read LDS and multiply; P producer waves issue every direct load of a stage
// (rows first, then weight blocks, spread evenly).  A wave that both issues a stage's loads and
// multiplies serialises the two: issuing stalls while the memory pipeline is full, and the
// MFMAs of that SIMD wait behind it.  With separate producer waves (one per SIMD for P = 4) the
// multiplies of stage i run while the loads of stage i+NBUF-1 issue.  Both kinds of wave pass
// the same barrier per stage: a producer refills slot (i-1) % NBUF only after every consumer
// finished reading it (its reads end with lgkmcnt(0) before the consumer reaches barrier i).
// ---------------------------------------------------------------------------------------------
__device__ __attribute__((aligned(16))) uint4 k44_t64_zero_row[8];  // 128 zero bytes

constexpr int T64R_IDX_MAX = 4096;

__device__ __forceinline__ uint32_t t64_lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

template <int NBK, int TW, int NBUF, int P>
__global__ __launch_bounds__(64 * (NBK * TW + P)) void k44_token64_ring_kernel(Token64Args a) {
    constexpr int NB = 4;                       // 16-neuron blocks per consumer wave
    constexpr int NC = NBK * TW;                // consumer waves
    constexpr int XST = 32 * 128;               // bytes of one tile's stage: 32 rows x 64 tokens
    constexpr int WST = NBK * NB * 1024;        // bytes of one stage's A fragments
    constexpr int SLOT = TW * XST + WST;
    constexpr int RP = 4 * TW / P, WP = 4 * NBK / P;  // row / weight loads per producer per stage
    static_assert(RP * P == 4 * TW && WP * P == 4 * NBK, "P divides the row and weight loads");
    constexpr int DP = RP + WP;
    __shared__ __attribute__((aligned(16))) char ring[NBUF][SLOT];
    extern __shared__ uint32_t ix[];  // B entries (dynamic: sized by the launch)

    const int tid = (int)threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Workgroup p runs on XCD p % 8.  The workgroups of one cluster gather the same rows: when
    // the grid allows, they are placed 8 apart (p = 8 * (bpc * q + h) + r holds block h of
    // cluster 8q + r), so they share one XCD's L2 instead of each XCD fetching the rows.  The
    // tile groups of one block (blockIdx.y) are gridDim.x apart: the same XCD whenever gridDim.x
    // is a multiple of 8, so they share the block's weights through that L2.
    uint32_t bx = blockIdx.x;
    {
        const uint32_t bpc = a.cluster / (64u * NBK);  // workgroups per cluster
        if (bpc > 1u && gridDim.x % (8u * bpc) == 0u) {
            const uint32_t r = bx & 7u, rest = bx >> 3, h = rest % bpc, q = rest / bpc;
            bx = bpc * (8u * q + r) + h;
        }
    }
    const uint32_t jw = bx * 64u * NBK;  // first neuron of the workgroup
    const uint32_t B = a.B_vec16 * 16u, ksteps = B / 32u;
    const uint32_t *irow = a.idx + (uint64_t)(jw / a.cluster) * B;
    for (uint32_t q = (uint32_t)tid; q < B; q += 64u * (NC + P)) {
        const uint32_t v = irow[q];
        ix[q] = v < a.Cin ? v : 0xffffffffu;
    }
    __syncthreads();
    const int gr = lane >> 3, gc = (lane & 7) * 16;  // row within an 8-row piece, byte column

    if (wave >= NC) {
        // Producer pw: row loads r = pw + P*m (piece r % 4 of tile r / 4 of the group), weight
        // blocks b = pw + P*m.
        const int pw = wave - NC;
        const char *zrow = reinterpret_cast<const char *>(k44_t64_zero_row) + gc;
        const uint64_t wblk = (uint64_t)a.B_vec16 * 32u * 16u;  // bytes of one 16-neuron block
        const char *xrow[RP];
        uint32_t ldsx[RP], ixa[RP];
#pragma unroll
        for (int m = 0; m < RP; ++m) {
            const int r = pw + P * m;
            const uint32_t t = blockIdx.y * TW + (uint32_t)(r / 4);
            xrow[m] = reinterpret_cast<const char *>(a.X + (uint64_t)t * a.Cin * 64u) + gc;
            ldsx[m] = (uint32_t)((r / 4) * XST + (r % 4) * 1024);
            ixa[m] = t64_lds_addr(&ix[8 * (r % 4) + gr]);
        }
        const char *wsrc = reinterpret_cast<const char *>(a.w_wmma) +
                           (uint64_t)(jw / 16u + (uint32_t)pw) * wblk + lane * 16;
        auto load_stage = [&](uint32_t ks, int buf) {
            uint32_t v[RP];
#pragma unroll
            for (int m = 0; m < RP; ++m)
                asm volatile("ds_read_b32 %0, %1" : "=v"(v[m]) : "v"(ixa[m] + ks * 128u) : "memory");
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            // The index words are used only after the wait (inline-asm reads are invisible to
            // the compiler's own wait insertion: without this it may compute addresses first).
#pragma unroll
            for (int m = 0; m < RP; ++m) asm volatile("" : "+v"(v[m]));
#pragma unroll
            for (int m = 0; m < RP; ++m) {
                const char *src = v[m] != 0xffffffffu ? xrow[m] + (uint64_t)v[m] * 128u : zrow;
                __builtin_amdgcn_global_load_lds(
                    (kglobal_void *)src, (__attribute__((address_space(3))) void *)&ring[buf][ldsx[m]],
                    16, 0, 2);  // non-temporal: gathered rows are not read again
            }
#pragma unroll
            for (int m = 0; m < WP; ++m) {
                const int b = pw + P * m;
                __builtin_amdgcn_global_load_lds(
                    (kglobal_void *)(wsrc + (uint64_t)(P * m) * wblk + (uint64_t)ks * 1024u),
                    (__attribute__((address_space(3))) void *)&ring[buf][TW * XST + b * 1024], 16, 0,
                    0);
            }
        };
        lds_ring<NBUF, DP>(ksteps, load_stage, [](int) {});
        return;
    }

    const int wt = wave % TW, wb = wave / TW;  // tile and 64-neuron block of this consumer
    const uint32_t j0 = jw + 64u * (uint32_t)wb;
    const uint32_t tile = blockIdx.y * TW + (uint32_t)wt;
    const int g = lane >> 4;
    f4_t acc[NB][4];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        f4_t b0 = {0.0f, 0.0f, 0.0f, 0.0f};
        if (a.bias) {
#pragma unroll
            for (int i = 0; i < 4; ++i) b0[i] = __half2float(a.bias[j0 + 16u * nb + 4u * g + i]);
        }
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) acc[nb][tb] = b0;
    }
    const int tr_row = 8 * g + ((lane & 15) >> 2), tr_col = 4 * (lane & 3);
    const uint32_t xa = t64_lds_addr(&ring[0][wt * XST + tr_row * 128 + tr_col * 2]);
    const uint32_t wa = t64_lds_addr(&ring[0][TW * XST + wb * NB * 1024 + lane * 16]);
    auto compute = [&](int buf) {
        const uint32_t x0 = xa + (uint32_t)buf * SLOT, w0 = wa + (uint32_t)buf * SLOT;
        h8_t af[NB];
        h4_t lo[4], hi[4];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
            asm volatile("ds_read_b128 %0, %1" : "=v"(af[nb]) : "v"(w0 + nb * 1024u) : "memory");
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(lo[tb]) : "v"(x0 + 32u * tb) : "memory");
            asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(hi[tb]) : "v"(x0 + 32u * tb + 512u)
                         : "memory");
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) asm volatile("" : "+v"(af[nb]));
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            asm volatile("" : "+v"(lo[tb]), "+v"(hi[tb]));
            const h8_t b = __builtin_shufflevector(lo[tb], hi[tb], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                acc[nb][tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[nb], b, acc[nb][tb], 0, 0, 0);
        }
    };
    lds_ring<NBUF, 1>(ksteps, [](uint32_t, int) {}, compute);

    // C layout: lane holds C[4g + i][lane & 15] of every 16x16 tile; round toward zero.
    __half *yt = a.Y + ((uint64_t)tile * a.Cout + j0) * 64u + (lane & 15);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2)
#pragma unroll
            for (int tb = 0; tb < 4; ++tb)
                yt[(uint64_t)(16 * nb + 4 * g + i2) * 64u + 16u * tb] =
                    __float2half_rz(acc[nb][tb][i2]);
}

static bool token64_ring_base_ok(const Token64Args &a) {
    return a.B_vec16 % 2u == 0u && a.B_vec16 * 16u <= (uint32_t)T64R_IDX_MAX;
}
// 128-neuron x 2-tile workgroups (both 64-neuron blocks share every gathered row).
static bool token64_ring128_ok(const Token64Args &a) {
    return token64_ring_base_ok(a) && a.cluster % 128u == 0u && a.tiles % 2u == 0u;
}
// 64-neuron x 4-tile workgroups.
static bool token64_ring_ok(const Token64Args &a) {
    return token64_ring_base_ok(a) && a.cluster % 64u == 0u && a.tiles % 4u == 0u;
}

hipError_t launch_token64(const Token64Args &a, hipStream_t stream, int ring_mode) {
    const size_t ix_bytes = (size_t)a.B_vec16 * 16u * 4u;
    // One producer wave per SIMD (P = 4): one, two and eight producers measured 25.7, 21.9 and
    // 21.7 us against 21.4 at the whitepaper shape; a 6-stage ring 21.8-22.0.
    if (ring_mode != 0 && ring_mode != 1 && token64_ring128_ok(a)) {
        const dim3 grid(a.Cout / 128u, a.tiles / 2u, 1u), block(64u * (4u + 4u), 1u, 1u);
        hipLaunchKernelGGL((k44_token64_ring_kernel<2, 2, 4, 4>), grid, block, ix_bytes, stream, a);
        return hipGetLastError();
    }
    if (ring_mode != 0 && ring_mode != 2 && token64_ring_ok(a)) {
        const dim3 grid(a.Cout / 64u, a.tiles / 4u, 1u), block(64u * (4u + 4u), 1u, 1u);
        hipLaunchKernelGGL((k44_token64_ring_kernel<1, 4, 4, 4>), grid, block, ix_bytes, stream, a);
        return hipGetLastError();
    }
    const uint32_t c16 = a.cluster / 16u;
    const int nb = c16 % 4u == 0u ? 4 : (c16 % 2u == 0u ? 2 : 1);
    const dim3 grid(a.Cout / (16u * (uint32_t)nb), (a.tiles + 3u) / 4u, 1u), block(256u, 1u, 1u);
    if (nb == 4)
        hipLaunchKernelGGL(k44_token64_kernel<4>, grid, block, 0, stream, a);
    else if (nb == 2)
        hipLaunchKernelGGL(k44_token64_kernel<2>, grid, block, 0, stream, a);
    else
        hipLaunchKernelGGL(k44_token64_kernel<1>, grid, block, 0, stream, a);
    return hipGetLastError();
}

// dst[g] = src[((tile / B_vec16) * 16 + (l & 15)) * B_vec8 + 2 * (tile % B_vec16) + (l >> 4)],
// tile = g / 32, l = g % 32: the WMMA vector order of a row-major [n][8*B_vec8] fp16 matrix
// (k44_plan_types.hpp:363-394; GPU form kernel44_immutable.cuh:261-267).  Grid-stride, 64-bit.
__global__ __launch_bounds__(256) void k44_interleave_wmma_kernel(uint4 *dst, const uint4 *src,
                                                                  uint64_t n_vec, uint32_t B_vec8) {
    const uint64_t B_vec16 = B_vec8 / 2u;
    for (uint64_t gi = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; gi < n_vec;
         gi += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t t = gi >> 5, l = gi & 31u;
        dst[gi] = src[((t / B_vec16) * 16u + (l & 15u)) * B_vec8 + 2u * (t % B_vec16) + (l >> 4)];
    }
}

hipError_t launch_interleave_wmma(uint4 *dst, const uint4 *src, uint32_t neurons, uint32_t B_vec8,
                                  hipStream_t stream) {
    const uint64_t n_vec = (uint64_t)(neurons / 16u) * (B_vec8 / 2u) * 32u;
    if (n_vec == 0u) return hipSuccess;
    const uint64_t blocks = std::min<uint64_t>((n_vec + 255u) / 256u, 65536u);
    hipLaunchKernelGGL(k44_interleave_wmma_kernel, dim3((uint32_t)blocks), dim3(256u), 0, stream,
                       dst, src, n_vec, B_vec8);
    return hipGetLastError();
}

}  // namespace k44dev
