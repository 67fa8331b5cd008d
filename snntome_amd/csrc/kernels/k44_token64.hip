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
// LDS-ring variant for the large shapes: clusters of a multiple of 64 neurons, batches of whole
// groups of 4 tiles, even B_vec16 (whole 32-deep k-steps), B <= 4096.  Workgroup = 64 neurons x
// 4 tiles (4 waves, one tile each).  The cluster's index row is staged in LDS once; then every
// k-step's 32 gathered rows per tile (128 B each: one global_load_lds_dwordx4 covers 8 rows) and
// its 64-neuron A fragments (1 KiB per 16-neuron block, contiguous in the WMMA order: one
// dwordx4 direct load per wave) go memory -> LDS directly, into a ring of 4 stages with 3 in
// flight (a 6-deep ring measured the same), synchronised exactly as the dense-cluster LDS-ring
// kernel (lds_ring, k44_mfma_dma.hpp):
// per stage vmcnt(2D) + bare s_barrier, LDS reads in inline asm with an explicit lgkmcnt wait.
// Rows of out-of-range indices are read from a zero row in device memory.
// ---------------------------------------------------------------------------------------------
__device__ __attribute__((aligned(16))) uint4 k44_t64_zero_row[8];  // 128 zero bytes

constexpr int T64R_IDX_MAX = 4096;

__device__ __forceinline__ uint32_t t64_lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// NBK 64-neuron blocks of one cluster per workgroup (1, or 2 when the cluster is a multiple of
// 128 neurons: both blocks then share every gathered row), 4 tiles, 4 * NBK waves: wave w owns
// tile w % 4 and block w / 4; the NBK waves of a tile split its row loads, every wave loads one
// 16-neuron block of A fragments per stage.
template <int NBK, int NBUF>
__global__ __launch_bounds__(256 * NBK) void k44_token64_ring_kernel(Token64Args a) {
    constexpr int NB = 4, TW = 4;
    constexpr int XST = 32 * 128;          // bytes of one tile's stage: 32 rows x 64 tokens x fp16
    constexpr int WST = NBK * NB * 64 * 16;  // bytes of one stage's A fragments
    constexpr int XR = 4 / NBK;            // 8-row loads per wave per stage
    constexpr int D = XR + 1;              // direct loads per wave per stage
    __shared__ __attribute__((aligned(16))) char xr[NBUF][TW][XST];
    __shared__ __attribute__((aligned(16))) char wr[NBUF][WST];
    extern __shared__ uint32_t ix[];  // B entries (dynamic: sized by the launch)

    const int tid = (int)threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wt = wave % TW, wb = wave / TW;  // tile and 64-neuron block of this wave
    // Workgroup p runs on XCD p % 8.  The workgroups of one cluster gather the same rows: when
    // the grid allows, they are placed 8 apart (p = 8 * (bpc * q + h) + r holds block h of
    // cluster 8q + r), so they share one XCD's L2 instead of each XCD fetching the rows.
    uint32_t bx = blockIdx.x;
    {
        const uint32_t bpc = a.cluster / (64u * NBK);  // workgroups per cluster
        if (bpc > 1u && gridDim.x % (8u * bpc) == 0u) {
            const uint32_t r = bx & 7u, rest = bx >> 3, h = rest % bpc, q = rest / bpc;
            bx = bpc * (8u * q + r) + h;
        }
    }
    const uint32_t jw = bx * 64u * NBK;  // first neuron of the workgroup
    const uint32_t j0 = jw + 64u * (uint32_t)wb;  // first neuron of this wave
    const uint32_t tile = blockIdx.y * TW + (uint32_t)wt;
    const uint32_t B = a.B_vec16 * 16u, ksteps = B / 32u;
    const uint32_t *irow = a.idx + (uint64_t)(jw / a.cluster) * B;
    for (uint32_t q = (uint32_t)tid; q < B; q += 256u * NBK) {
        const uint32_t v = irow[q];
        ix[q] = v < a.Cin ? v : 0xffffffffu;
    }
    __syncthreads();

    const char *xt = reinterpret_cast<const char *>(a.X + (uint64_t)tile * a.Cin * 64u);
    const char *zrow = reinterpret_cast<const char *>(k44_t64_zero_row);
    const int gr = lane >> 3, gc = (lane & 7) * 16;  // row within an 8-row piece, byte column
    // A fragments of 16-neuron block `wave` of the workgroup: WMMA vectors
    // (jw/16 + wave, 2 ks .. 2 ks + 1, 0..31), 1 KiB contiguous per k-step.
    const char *wsrc = reinterpret_cast<const char *>(a.w_wmma) +
                       ((uint64_t)(jw / 16u + (uint32_t)wave) * a.B_vec16 * 32u) * 16u;
    // This wave loads 8-row pieces p = wb * XR .. wb * XR + XR - 1 of its tile's stage.
    const uint32_t ix_addr = t64_lds_addr(&ix[8 * wb * XR + gr]);

    auto load_stage = [&](uint32_t ks, int buf) {
        uint32_t v[XR];
        const uint32_t base = ix_addr + ks * 128u;
        if constexpr (XR == 4)
            asm volatile("ds_read_b32 %0, %4\n\tds_read_b32 %1, %4 offset:32\n\t"
                         "ds_read_b32 %2, %4 offset:64\n\tds_read_b32 %3, %4 offset:96\n\t"
                         "s_waitcnt lgkmcnt(0)"
                         : "=v"(v[0]), "=v"(v[1]), "=v"(v[2]), "=v"(v[3]) : "v"(base) : "memory");
        else
            asm volatile("ds_read_b32 %0, %2\n\tds_read_b32 %1, %2 offset:32\n\t"
                         "s_waitcnt lgkmcnt(0)"
                         : "=v"(v[0]), "=v"(v[1]) : "v"(base) : "memory");
#pragma unroll
        for (int i = 0; i < XR; ++i) {
            const char *src = v[i] != 0xffffffffu ? xt + (uint64_t)v[i] * 128u + gc : zrow + gc;
            __builtin_amdgcn_global_load_lds(
                (kglobal_void *)src,
                (__attribute__((address_space(3))) void *)&xr[buf][wt][(wb * XR + i) * 1024], 16, 0,
                0);
        }
        __builtin_amdgcn_global_load_lds((kglobal_void *)(wsrc + (uint64_t)ks * 1024u + lane * 16),
                                         (__attribute__((address_space(3))) void *)&wr[buf][wave * 1024],
                                         16, 0, 0);
    };

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
    const uint32_t xa = t64_lds_addr(&xr[0][wt][tr_row * 128 + tr_col * 2]);
    const uint32_t wa = t64_lds_addr(&wr[0][wb * NB * 1024 + lane * 16]);
    auto compute = [&](int buf) {
        const uint32_t x0 = xa + (uint32_t)buf * (TW * XST), w0 = wa + (uint32_t)buf * WST;
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

    lds_ring<NBUF, D>(ksteps, load_stage, compute);

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

bool token64_ring_ok(const Token64Args &a) {
    return a.cluster % 64u == 0u && a.tiles % 4u == 0u && a.B_vec16 % 2u == 0u &&
           a.B_vec16 * 16u <= (uint32_t)T64R_IDX_MAX;
}

hipError_t launch_token64(const Token64Args &a, hipStream_t stream, int ring_mode) {
    if (token64_ring_ok(a) && ring_mode != 0) {
        // Two 64-neuron blocks sharing every gathered row: half the row traffic but half the
        // workgroups; measured equal at 128-neuron clusters, slightly faster from 256 on.
        const size_t ix_bytes = (size_t)a.B_vec16 * 16u * 4u;
        if (a.cluster % 256u == 0u && ring_mode != 1) {
            const dim3 grid(a.Cout / 128u, a.tiles / 4u, 1u), block(512u, 1u, 1u);
            hipLaunchKernelGGL((k44_token64_ring_kernel<2, 6>), grid, block, ix_bytes, stream, a);
        } else {
            // (A 3-stage ring, two workgroups per CU, measured 3 % slower at the whitepaper shape.)
            const dim3 grid(a.Cout / 64u, a.tiles / 4u, 1u), block(256u, 1u, 1u);
            hipLaunchKernelGGL((k44_token64_ring_kernel<1, 4>), grid, block, ix_bytes, stream, a);
        }
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
