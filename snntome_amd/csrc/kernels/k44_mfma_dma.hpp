// k44_mfma_dma.hpp — MFMA dense-cluster wave kernel with an LDS ring filled by direct loads.
//
// Same contraction and epilogue as k44_mfma_tile_kernel (Y[NT][512 tokens] = W[NT][K*S] x
// X_gathered[K*S][512] on v_mfma_f32_16x16x32_f16), for the shape that carries the large
// waves: 512 tokens per workgroup (8 waves x 64 tokens), NT in {32, 64, 128}.
//
// What differs is how data reaches LDS.  The register-staged kernel keeps one stage of X in
// flight per workgroup (its loads must land in registers before they can be stored to LDS), so
// it is bound by memory latency, not bandwidth.  Here every stage of 32 positions goes straight
// from memory to LDS with global_load_lds (gfx950): each X row of 512 tokens is one
// global_load_lds_dwordx4 (64 lanes x 16 bytes = the whole 1 KiB row, written at the row's
// padded LDS pitch), and the stage's A fragments (64*NT bytes, contiguous in the upload order)
// are NT/32 global_load_lds_dword per wave.  A ring of NBUF = 4 stages keeps 3 stages
// (~113 KiB) of the CU's one workgroup in flight while the 4th is multiplied (gathers from
// HBM); NBUF = 2 (74 KiB of LDS) fits two workgroups per CU, each with one stage in flight
// (gathers that hit the caches).  No staging registers, no ds_write.
//
// Synchronisation per stage i (every wave issues the same D = 4 + NT/32 loads per stage;
// shown for NBUF = 4):
//   s_waitcnt vmcnt(2D) lgkmcnt(0)   own loads of stage i landed; own LDS reads of i-1 done
//   s_barrier                        every wave's loads of stage i landed; nobody reads i-1
//   issue stage i+3 into ring slot (i+3)%4 = (i-1)%4
//   MFMAs of stage i from slot i%4
// The last three stages drain with vmcnt(2D), vmcnt(D), vmcnt(0).  The waits are explicit
// because a workgroup barrier with a memory fence (__syncthreads) would wait for every load in
// flight; compiler barriers keep LDS accesses on their side of each s_barrier.
#pragma once
#include "k44_mfma_tile.hpp"

namespace k44dev {

// s_waitcnt vmcnt(N) lgkmcnt(0) (gfx9 encoding: vmcnt[3:0] + vmcnt[5:4] at bits 15:14,
// expcnt[6:4] left at its maximum, lgkmcnt[11:8] = 0).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

__device__ __forceinline__ void wg_barrier_no_fence() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Drain of an LDS ring: R stages left, all issued; each waits for its own loads with the
// younger ones still in flight.
template <int R, int NBUF, int D, typename Comp>
__device__ __forceinline__ void lds_ring_drain(uint32_t left, uint32_t &i, Comp &comp) {
    if constexpr (R >= 1) {
        if (left == (uint32_t)R) {
            wait_vm_lgkm0<(R - 1) * D>();
            wg_barrier_no_fence();
            comp((int)(i % NBUF));
            ++i;
            --left;
        }
        lds_ring_drain<R - 1, NBUF, D>(left, i, comp);
    }
}

// Schedule of an LDS ring of NBUF stages with NBUF-1 in flight, D direct loads per wave per
// stage: load(stage, slot) issues a stage's direct loads into ring slot `slot`, comp(slot)
// multiplies a landed stage.  Stage i is multiplied after (a) this wave's loads of stage i have
// landed — the loads of the NBUF-2 younger stages may still be in flight: vmcnt((NBUF-2)·D) —
// and (b) a barrier, after which every wave's loads of stage i have landed and no wave still
// reads slot (i-1) % NBUF, which stage i+NBUF-1 then refills.  The last NBUF-1 stages drain
// with decreasing vmcnt.  n_st >= 1.
template <int NBUF, int D, typename Load, typename Comp>
__device__ __forceinline__ void lds_ring(uint32_t n_st, Load &&load, Comp &&comp) {
    constexpr int AHEAD = NBUF - 1;
#pragma unroll
    for (int p = 0; p < AHEAD; ++p)
        if ((uint32_t)p < n_st) load((uint32_t)p, p);
    uint32_t i = 0;
    for (; i + AHEAD < n_st; ++i) {
        wait_vm_lgkm0<(AHEAD - 1) * D>();
        wg_barrier_no_fence();
        load(i + AHEAD, (int)((i + AHEAD) % NBUF));
        comp((int)(i % NBUF));
    }
    lds_ring_drain<AHEAD, NBUF, D>(n_st - i, i, comp);
}

// Byte address of a shared-memory location in the LDS aperture.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

__device__ __forceinline__ h8_t ds_read_b128_at(uint32_t addr) {
    h8_t v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr) : "memory");
    return v;
}

// ds_read_b64_tr_b16: 4 x 16-bit, transposed across each 16-lane group (see lds_read_tr16).
__device__ __forceinline__ h4_t ds_read_tr16_at(uint32_t addr) {
    h4_t v;
    asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(v) : "v"(addr) : "memory");
    return v;
}

// NTX: the direct loads use the non-temporal cache policy (substrates far beyond the caches).
// NT = 128 (a 128-neuron tile: twice the MFMA work per gathered stage; 128 accumulator registers
// per lane, so one workgroup per CU) takes a 3-stage ring (125 KiB of LDS, 2 stages in flight).
//
// P > 0: producer and consumer waves.  The 8 waves above stop issuing loads and only read LDS,
// multiply and run the epilogue (consumers); P more waves (producers) issue every direct load of
// a stage: ROWS / P row loads and NT / (16 P) A-fragment loads of 1 KiB (dwordx4) each.  A wave
// that both issues a stage's loads and multiplies serialises the two (issuing stalls while the
// memory pipeline is full, and its SIMD's MFMAs wait behind it); with the roles split the
// multiplies of stage i run while the loads of stage i+NBUF-1 issue.  Both roles pass the same
// barrier per stage (a producer refills a slot only after every consumer's reads of it
// completed); the producers then end, and the epilogue's barrier waits for the consumers only
// (s_barrier counts the waves of the workgroup that have not ended).
template <int NT, bool NTX, int NBUF = 4, int P = 0>
__global__ __launch_bounds__(512 + 64 * P) void k44_mfma_dma_kernel(K44_GROUP_PARAMS) {
    K44_GROUP_BIND;
    static_assert(NT == 32 || NT == 64 || NT == 128,
                  "A-fragment stage must be whole dword loads per wave");
    static_assert(P == 0 || ((32 % P) == 0 && ((NT / 16) % P) == 0),
                  "producers split the row and A-fragment loads evenly");
    constexpr int MT = 512, ROWS = 32;
    constexpr int NB = NT / 16;
    constexpr int PITCH = MT + 16;          // halves; 32-byte skew between rows
    constexpr int WBYTES = NT * ROWS * 2;   // A fragments of one stage
    constexpr int WDMA = WBYTES / (8 * 256);  // dword loads per wave per stage (NT / 32)
    constexpr int XDMA = ROWS / 8;          // row loads per wave per stage
    constexpr int D = XDMA + WDMA;          // loads per wave per stage
    constexpr int CPOL = NTX ? 2 : 0;       // cache-policy operand: 2 = nt
    __shared__ __attribute__((aligned(16))) _Float16 xl[NBUF][ROWS][PITCH];
    __shared__ __attribute__((aligned(16))) uint32_t wl[NBUF][WBYTES / 4];
    static_assert(sizeof(xl) >= 8 * EPI_WAVE_FLOATS * sizeof(float), "epilogue LDS regions");

    uint32_t w;
    const uint32_t item = group_item_wave(grp, w);
    const MfmaTileArgs a = grp.waves[w];
    const uint32_t local = item - grp.start[w];
    const uint32_t tile = local % a.tiles, rest = local / a.tiles;
    const uint32_t ytile = rest % a.ttiles, zgroup = rest / a.ttiles;

    const int tid = (int)threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t tok0 = ytile * (uint32_t)MT;
    // Segment starts are read-only for the kernel's lifetime: scalar loads.
    const kconst_u64 *segr = (const kconst_u64 *)(a.seg) + (uint64_t)tile * a.K;
    const uint32_t stages = a.K * a.S / (uint32_t)ROWS;
    const uint32_t st_begin = zgroup * a.stage_chunk;
    const uint32_t st_end = min(stages, st_begin + a.stage_chunk);
    const uint32_t n_st = st_end - st_begin;
    // A fragments of the tile: [k-step][16-neuron block][lane][8 halves]; one stage = one k-step.
    const char *wtile = reinterpret_cast<const char *>(a.Wf) + (uint64_t)tile * a.ksteps * WBYTES;

    // This lane's 8 tokens of every gathered row (the same offset for every stage).
    const uint64_t lane_x = tok_x(a, tok0 + (uint32_t)lane * 8u);
    auto issue = [&](uint32_t st, int buf) {
        const uint32_t kk = st * (uint32_t)ROWS;
        const uint32_t k = kk / a.S, s0 = kk - k * a.S;
        const __half *base = a.X + segr[k] + (uint64_t)s0 * a.step + lane_x;
#pragma unroll
        for (int r = 0; r < XDMA; ++r) {
            const int row = wave + 8 * r;
            __builtin_amdgcn_global_load_lds((kglobal_void *)(base + (uint64_t)row * a.step),
                                             (__attribute__((address_space(3))) void *)&xl[buf][row][0],
                                             16, 0, CPOL);
        }
        const char *ws = wtile + (uint64_t)st * WBYTES;
#pragma unroll
        for (int j = 0; j < WDMA; ++j) {
            const int q = wave * WDMA + j;  // 256-byte piece of the stage's A fragments
            __builtin_amdgcn_global_load_lds((kglobal_void *)(ws + q * 256 + lane * 4),
                                             (__attribute__((address_space(3))) void *)&wl[buf][q * 64],
                                             4, 0, CPOL);
        }
    };

    f4_t acc[NB][4];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) acc[nb][tb] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int g = lane >> 4;
    const int tr_row = 8 * g + ((lane & 15) >> 2);  // row read by this lane (first half)
    const int tr_col = wave * 64 + 4 * (lane & 3);  // token column (+16 per token block)
    // LDS reads of a stage are inline asm: the compiler would otherwise make every LDS read
    // wait for all direct loads in flight (it cannot tell the ring slots apart), which would
    // serialise the ring.  Their completion is awaited explicitly before the MFMAs.
    const uint32_t xa = lds_addr(&xl[0][tr_row][tr_col]);
    const uint32_t wa = lds_addr(&wl[0][lane * 4]);
    constexpr uint32_t XBUF = ROWS * PITCH * 2, WBUF = WBYTES;
    auto compute = [&](int buf) {
        const uint32_t x0 = xa + (uint32_t)buf * XBUF, w0 = wa + (uint32_t)buf * WBUF;
        h8_t af[NB];
        h4_t lo[4], hi[4];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) af[nb] = ds_read_b128_at(w0 + nb * 1024u);
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            lo[tb] = ds_read_tr16_at(x0 + 32u * tb);
            hi[tb] = ds_read_tr16_at(x0 + 32u * tb + 8u * PITCH);
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

    if constexpr (P == 0) {
        lds_ring<NBUF, D>(n_st, [&](uint32_t st, int buf) { issue(st_begin + st, buf); }, compute);
    } else if (wave >= 8) {
        // Producer pw: rows pw + P*r of every stage, A-fragment blocks pw + P*j.
        constexpr int RP = ROWS / P, WP = NB / P;
        const int pw = wave - 8;
        const __half *xlane = a.X + lane_x;
        const char *wlane = wtile + (uint64_t)pw * 1024u + (uint32_t)lane * 16u;
        auto pissue = [&](uint32_t st, int buf) {
            const uint32_t kk = st * (uint32_t)ROWS;
            const uint32_t k = kk / a.S, s0 = kk - k * a.S;
            const __half *base = xlane + segr[k] + (uint64_t)(s0 + (uint32_t)pw) * a.step;
#pragma unroll
            for (int r = 0; r < RP; ++r)
                __builtin_amdgcn_global_load_lds(
                    (kglobal_void *)(base + (uint64_t)(P * r) * a.step),
                    (__attribute__((address_space(3))) void *)&xl[buf][pw + P * r][0], 16, 0, CPOL);
            const char *ws = wlane + (uint64_t)st * WBYTES;
#pragma unroll
            for (int j = 0; j < WP; ++j)
                __builtin_amdgcn_global_load_lds(
                    (kglobal_void *)(ws + (uint32_t)(P * j) * 1024u),
                    (__attribute__((address_space(3))) void *)&wl[buf][(pw + P * j) * 256], 16, 0,
                    CPOL);
        };
        lds_ring<NBUF, RP + WP>(n_st, [&](uint32_t st, int buf) { pissue(st_begin + st, buf); },
                                [](int) {});
        return;
    } else {
        lds_ring<NBUF, 1>(n_st, [](uint32_t, int) {}, compute);
    }

    // Every wave is done with the ring (its LDS reads completed) before the LDS-transposed
    // epilogue reuses the X slots.
    if (a.epi_vec) wg_barrier_no_fence();
    mfma_tile_epilogue<NT>(a, acc, tile, tok0, zgroup, lane, wave,
                           reinterpret_cast<float *>(&xl[0][0][0]) + wave * EPI_WAVE_FLOATS);
}

}  // namespace k44dev
