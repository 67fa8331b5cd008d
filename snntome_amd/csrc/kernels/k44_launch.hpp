// k44_launch.hpp — host-side launchers of the wave kernels (one translation unit per kernel
// family, compiled in parallel; see kernels/*.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "k44_gather_dot.hpp"
#include "k44_mfma_tile.hpp"
#include "k44_aux.hpp"

namespace k44dev {

// VALU gather-dot over `cout` neurons x `tokens` tokens with the given slab (64/128/256);
// ksplit 4 = one neuron per workgroup, its segments split over the 4 waves.
// lane8: 8 tokens (16-byte loads) per lane instead of 4 (8-byte loads); same weight layout.
// Streaming gather kernel (256-token slabs, no residual): output rows staged in LDS and written
// after the workgroup's last gather.  tokens: a multiple of 256.
hipError_t launch_gather_stream(const GatherDotArgs &a, uint32_t tokens, hipStream_t stream,
                                bool stream_loads);
// stream_loads: read X rows and weights with non-temporal loads (substrates far beyond the caches).
// weights_in_lds: the 8-token kernel stages each neuron's weights in LDS when they fit (false:
// read per 16-row batch; same values and FMA order).
// misaligned: segment starts at any element (4-token lanes only; lane8 must be false).
hipError_t launch_gather_dot(const GatherDotArgs &a, uint32_t slab, uint32_t ksplit,
                             uint32_t tokens, hipStream_t stream, bool lane8 = false,
                             bool stream_loads = false, bool weights_in_lds = true,
                             bool misaligned = false);

// MFMA tile kernel over a group of waves (one kernel configuration): `items` workgroups (the
// group's start[n]), block mt; nt in {16,32,64,128}, mt in {64,128,256,512}, rows_per_stage in
// {32,64}.  mis: segment rows at any element offset (shifted into place; rows_per_stage 32).
hipError_t launch_mfma_tile(const MfmaGroup &g, uint32_t nt, uint32_t mt, uint32_t rows_per_stage,
                            uint32_t items, hipStream_t stream, bool mis = false);

// Shape of an LDS-DMA MFMA launch: ring stages (4: one workgroup per CU, 3 stages in flight;
// 2: two workgroups per CU, 1 stage in flight each; 3: 128-neuron tiles, one workgroup per CU,
// 2 stages in flight) and the loads' cache policy.
struct DmaShape {
    uint32_t nbuf = 4;
    bool stream_loads = false;
    uint32_t prod = 0;  // producer waves (0: every wave loads and multiplies)
    bool operator==(const DmaShape &o) const {
        return nbuf == o.nbuf && stream_loads == o.stream_loads && prod == o.prod;
    }
};

// LDS-DMA MFMA tile kernel (512 tokens per workgroup, 32-position stages through an LDS ring
// filled by direct loads) over a group: `items` workgroups; nt in {32, 64} (2 or 4 stages) or
// 128 (3 stages).
hipError_t launch_mfma_dma(const MfmaGroup &g, uint32_t nt, uint32_t items, hipStream_t stream,
                           const DmaShape &shape);

// Narrow MFMA kernel (waves of at most 16 tokens) over a group: `items` workgroups (tiles x
// contraction chunks per wave); nt in {16,32,64,128}.  prod: 0, or the element-wise product
// form (MfmaTileArgs::xprod 2 / 3) every wave of the group gathers (nt 64 / 128 only).
// max_items: the largest wave's workgroups (nt 64 / 128 take a (max_items x waves) grid when
// that wastes little).  pre: up to six waves' weights and geometry as kernel arguments (nt 64
// / 128; zero entries: read from the descriptors).
hipError_t launch_mfma_narrow(const MfmaGroup &g, uint32_t nt, uint32_t items, hipStream_t stream,
                              uint32_t prod = 0, uint32_t max_items = 0,
                              const NarrowPre &pre = NarrowPre{});

// out[b] = the XCD workgroup b of an n-workgroup launch ran on (set-up check of the narrow
// kernels' XCD-local split-K meeting).
hipError_t launch_xcd_probe(uint32_t *out, uint32_t n, hipStream_t stream);

// Split-K second pass over the same group: grid epi_max x g.n (epi_max = the largest wave's
// epilogue workgroups, ceil(cout * tokens / 4 / 256); 0: no wave of the group is split).
hipError_t launch_splitk_epilogue(const MfmaGroup &g, uint32_t epi_max, hipStream_t stream);

// Stand-alone Token64 wave (X [tiles][Cin][64], Y [tiles][Cout][64], per-cluster index rows,
// RDNA4-WMMA-ordered weights, bias, round toward zero); see k44_token64.hip.
struct Token64Args {
    __half *Y;
    const __half *X;
    const uint32_t *idx;   // [Cout / cluster][16 * B_vec16] input positions
    const uint4 *w_wmma;   // [Cout / 16][B_vec16][32] vectors of 8 fp16
    const __half *bias;    // [Cout] or nullptr (zero)
    uint32_t Cin, Cout, B_vec16, cluster, tiles;
};
// ring_mode: -1 automatic, 0 per-wave kernel, 1 only the 64-neuron x 4-tile ring kernel, 2 only
// the 128-neuron x 2-tile ring kernel (each where the shape allows it, else the per-wave kernel).
hipError_t launch_token64(const Token64Args &a, hipStream_t stream, int ring_mode = -1);

// GPU weight interleave: row-major [neurons][8 * B_vec8] fp16 -> WMMA vector order.
hipError_t launch_interleave_wmma(uint4 *dst, const uint4 *src, uint32_t neurons, uint32_t B_vec8,
                                  hipStream_t stream);

// Synthetic substrate fill (see k44_fill_uniform_kernel).
hipError_t launch_fill_uniform(__half *dst, uint64_t rows, uint32_t stride, uint32_t valid,
                               uint64_t pos0, uint64_t seed, hipStream_t stream);

}  // namespace k44dev
