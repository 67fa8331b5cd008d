// k44_mfma_tile.hpp — MFMA dense-cluster wave kernel for gfx950.
//
// For waves whose neurons come in tiles of NT (16..128) that share one index row ("cluster"
// in the reference's plan, k44_plan_types.hpp:167-186), and whose dendritic segments are
// multiples of 32 positions: the tile is a dense contraction
//     Y[NT neurons][M tokens] = W[NT][K*S] x X_gathered[K*S][M]
// fed to v_mfma_f32_16x16x32_f16 (fp16 in, fp32 accumulate).
//
// Data path (one workgroup = one neuron tile x MT tokens, MT/64 waves):
//  * X: each stage is ROWS consecutive substrate positions of one segment x MT tokens, read
//    from HBM with 16-byte loads (a position row is token-contiguous on the canvas) into
//    registers one stage ahead, then stored to LDS unchanged ([row][token], padded pitch).
//    The B operand needs 8 consecutive positions for one token per lane; ds_read_b64_tr_b16
//    delivers exactly that from the untransposed tile: lane 16g+4j+m reads row 8g+j (+4),
//    tokens t0+4m..+3, and after the transpose lane 16g+i holds positions 8g..8g+3 (+4..+7)
//    of token t0+i.  Two LDS buffers ping-pong; one barrier per stage.
//  * W: pre-arranged at upload in MFMA A-fragment order ([tile][k-step][16-neuron block]
//    [lane][8]), so each wave loads every A fragment with one coalesced 16-byte-per-lane load.
//  * Each wave owns 64 tokens: NT/16 x 4 accumulator tiles of 16x16 fp32.
//  * Epilogue fused: bias, activation, residual / cout_map, fp16 (RNE) store.
//  * Split-K for launches with too few tiles to fill the chip (decode-sized token counts, waves
//    of one or two tiles): grid.z workgroups share a tile, each runs a contiguous range of
//    stages and stores an fp32 partial; a second kernel reduces the partials in fixed order
//    (bit-reproducible) and runs the epilogue.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "k44_gather_dot.hpp"

namespace k44dev {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef short s4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u4_t __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16 on an LDS address: 4 x 16-bit, transposed across each 16-lane group.
__device__ __forceinline__ h4_t lds_read_tr16(const _Float16 *p) {
    const s4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s4_t *)(p));
    return __builtin_bit_cast(h4_t, v);
}

struct MfmaTileArgs {
    const __half *X;       // canvas base
    const uint64_t *seg;   // [rows][K] canvas element offset of each segment start
    const __half *Wf;      // A-fragment ordered weights
    const __half *bias;    // [cout] or nullptr
    const uint16_t *cmap;  // [cout] or nullptr
    __half *Y;             // canvas + y_off
    const __half *R;       // canvas + res_off or nullptr
    uint64_t step;         // canvas elements between consecutive positions of a segment
    uint32_t K, S;         // segments per row, positions per segment (S % ROWS == 0)
    uint32_t ksteps;       // K*S/32
    uint32_t out_stride;
    int act;
    // Split-K (part != nullptr): workgroup z covers stages [z*stage_chunk, +stage_chunk) and
    // stores its fp32 partial tile to part[(z*cout + j)*tokens + t]; k44_splitk_epilogue_kernel
    // sums the partials in z order and runs the epilogue.  part == nullptr: stage_chunk = all.
    float *part;
    uint32_t stage_chunk;
    uint32_t cout;    // neurons of the wave (partial row count)
    uint32_t tokens;  // tokens of the wave (partial row length)
    // Work items of the wave: tiles x token tiles x split-K groups (tile index fastest).
    uint32_t tiles, ttiles, kgroups;
    // Product gather (element-wise multiplies fused into the X gather; narrow kernels of 64 /
    // 128-neuron tiles only): xprod 0 = the X rows as they are; 2 = fp16(A*B); 3 =
    // fp16(A*fp16(B*C)), A / B / C the rows at (segment offset + xd[0] / xd[1] / xd[2]);
    // 4 = a folded RMSNorm of the rows at (segment offset + xd[0]) (fields below); 5 = the
    // same followed by the decode token shift of the normalised rows (fields below).
    uint32_t xprod;
    int64_t xd[3];
    // 2-D waves of 64-frame interleaved images: 64-token tile t of the wave gathers at
    // segment offset + tile_x[t] and stores at tile_y[t] (every entry 64-element aligned);
    // nullptr: 1-D token rows, tile t at 64 t for both.
    const uint32_t *tile_x, *tile_y;
    // 1: Y, R and out_stride are multiples of 8 elements (and split-K partial rows of 4), so
    // the epilogue may use 16-byte accesses (mfma_tile_epilogue_lds).
    uint32_t epi_vec;
    // Narrow kernels of 64 / 128-neuron tiles with split-K: per-tile arrival counters (zero
    // between launches).  The last workgroup of a tile to arrive sums the partials in chunk order
    // and runs the epilogue; partials are then laid out [z][cout/4][16 tokens][4 neurons].
    // nullptr: partials [z][cout][16] for k44_splitk_epilogue_kernel.
    uint32_t *arrive;
    // RMSNorm folded around narrow 64 / 128-neuron waves (whole-plan runs), producer side
    // (norm_part set): once a tile's outputs are stored, the tile stores the exact per-token sums
    // of squares of the fp16 values it stored (k44_sumsq.hpp) in its slot norm_part[tile]
    // (16 tokens x 2 words: limbs 0 | 1, limb 2 | inf / NaN flags).
    uint32_t *norm_part;
    uint32_t norm_D;  // consumer side: channels and epsilon of the norm
    float norm_eps;
    // Consumer side (xprod 4): the gather reads the norm's input rows (segment offset + xd[0])
    // and replaces every element by fp16(x * inv[t] * gamma[c]), the RMSNorm kernel's
    // expression; inv[t] = rsqrt(sum / norm_D + norm_eps) from the xslots_n producer slots at
    // xslots; gamma from xgamma (nullptr: 1), c = (row offset - xg_base) >> xg_shift.
    const uint32_t *xslots;
    uint32_t xslots_n;
    const __half *xgamma;
    uint64_t xg_base;
    uint32_t xg_shift;
    // xprod 5: each normalised element n of channel c, token t becomes the decode token shift's
    // output fp16(mu[c][0] n + sum_{i=1}^{rf-1} mu[c][i] state[c][i-1][t]) (the shift kernel's
    // expression) for t < sh_tokens, and 0 beyond.  The state is read from a compact copy
    // ([c][rf-1][16 tokens], refreshed from the plan's state by an earlier launch: 32 of every
    // 128 bytes of the plan's [c][rf-1][64] rows are the tokens).  The shifted state ([n,
    // state[c][0], .., state[c][rf-3]] for t < sh_tokens, unchanged beyond) cannot be stored in
    // place (other workgroups of the launch read the old state): the workgroup whose bit
    // own[item] has for a 32-row pass (bit sub-chunk * 16 + pass) stores it for the pass's
    // channels in state_next [c][rf-1][16], and a later launch copies it back (cp_* below).
    // 2 <= rf <= 4.
    const __half *mixg;        // [D][8]: mixing weights mu[c][0..rf-1] (0 past rf), the
                               // norm's gamma[c] (1 without one) at 4, 0 at 5..7
    const __half *state;       // [D][rf-1][16] (compact copy)
    __half *state_next;        // [D][rf-1][16]
    const uint64_t *own;       // [tiles * kgroups]
    uint32_t rf, sh_tokens;
    // Copy carried by this wave's workgroups (cp_rows 0: none): cp_rows rows of 16 fp16 from
    // cp_src + cp_sstride r to cp_dst + cp_dstride r (strides in elements): a folded token
    // shift's state refreshed into its compact copy before its readers, or its shifted state
    // copied back after them.
    const __half *cp_src;
    __half *cp_dst;
    uint32_t cp_rows, cp_sstride, cp_dstride;
    // Split-K reduced inside the launch through one XCD's L2 (red_local 1; arrive set): the
    // wave's work items are numbered so that the chunks of a tile are 8 apart in launch order
    // (position p: tile 8 (p / 8kg) + p % 8, chunk (p % 8kg) / 8; positions of tiles past the
    // wave's are idle), which the round-robin dispatch over the XCDs places on one XCD (set-up
    // checks it); the partials are then plain stores, the arrival counter an L2 atomic and the
    // reads L1-bypassing loads, instead of device-coherent accesses.
    uint32_t red_local;
    // Single-frame 2-D outputs whose 64-token tiles span plane rows (padded-plane layout, W not
    // a multiple of 64): token t of tile tl of its frame is pixel rel = 64 tl + (t & 63) of the
    // padded rows, stored only when rel / mask_wpad < mask_h and rel % mask_wpad < mask_w (the
    // halo columns stay as they are).  mask_w == 0: every token is stored.
    uint32_t mask_w, mask_h, mask_wpad, mask_tpf;
};

// Whether token t of a wave is stored (see MfmaTileArgs::mask_w).
__device__ __forceinline__ bool tok_stored(const MfmaTileArgs &a, uint32_t t) {
    if (!a.mask_w) return true;
    const uint32_t rel = 64u * ((t >> 6) % a.mask_tpf) + (t & 63u);
    const uint32_t row = rel / a.mask_wpad;
    return row < a.mask_h && rel - row * a.mask_wpad < a.mask_w;
}

// Eight consecutive fp16 elements m .. m+7 (m in 0..7) of the 16 held in lo:hi (two aligned
// 16-byte chunks): the dwords selected by m / 2 and, for odd m, funnel-shifted by 16 bits.
// Used for rows that start off the 16-byte grid (token-shifted taps), each lane with its own m.
__device__ __forceinline__ u4_t shift_elems(const u4_t &lo, const u4_t &hi, uint32_t m) {
    const uint32_t A[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    const uint32_t q = m >> 1;
    uint32_t d[5];
#pragma unroll
    for (int j = 0; j < 5; ++j)
        d[j] = q == 0u ? A[j] : q == 1u ? A[j + 1] : q == 2u ? A[j + 2] : A[j + 3];
    u4_t r;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        r[j] = (m & 1u) ? __builtin_amdgcn_alignbit(d[j + 1], d[j], 16u) : d[j];
    return r;
}

// Canvas offset of token t of a wave (relative to a segment row or an output row).
__device__ __forceinline__ uint64_t tok_x(const MfmaTileArgs &a, uint32_t t) {
    return a.tile_x ? (uint64_t)a.tile_x[t >> 6] + (t & 63u) : (uint64_t)t;
}
__device__ __forceinline__ uint64_t tok_y(const MfmaTileArgs &a, uint32_t t) {
    return a.tile_y ? (uint64_t)a.tile_y[t >> 6] + (t & 63u) : (uint64_t)t;
}

// A launch covers a group of independent waves of one kernel configuration (the sub-waves of a
// pruned projection, projections reading the same input): workgroup i belongs to the wave w with
// start[w] <= i < start[w+1]; the split-K epilogue runs grid (largest wave's epilogue
// workgroups) x (waves).
struct MfmaGroup {
    const MfmaTileArgs *waves;  // [n]
    const uint32_t *start;      // [n+1] prefix sums of tiles * ttiles * kgroups
    uint32_t n;
    uint32_t xcd_order;         // 0 plain, 1 contiguous per XCD, 2 per-wave shares (group_item_wave)
};

// Group kernels take the four MfmaGroup fields as separate scalar parameters: the build preloads
// leading scalar kernel arguments into SGPRs at dispatch (-amdgpu-kernarg-preload-count), while
// an aggregate parameter is read from the kernel-argument segment by a load every wave of the
// launch waits for before its first dependent (descriptor) load.
#define K44_GROUP_PARAMS \
    const MfmaTileArgs *grp_waves, const uint32_t *grp_start, uint32_t grp_n, uint32_t grp_xcd
#define K44_GROUP_ARGS(g) (g).waves, (g).start, (g).n, (g).xcd_order
#define K44_GROUP_BIND const MfmaGroup grp{grp_waves, grp_start, grp_n, grp_xcd}

// XCD (accelerator complex die) this wave runs on.
__device__ __forceinline__ uint32_t k44_xcc_id() {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    return v & 0xfu;
}

// Weights and contraction geometry of up to six waves of a narrow launch, passed as scalar
// kernel arguments (preloaded into SGPRs like the group fields), so that a workgroup issues
// its weight stream before its descriptor load has returned.  The waves' A fragments are
// copies in one buffer, wave m's at base + (m << shift); geo[m] packs tiles (10 bits),
// red_local (1), ksteps (8), stage_chunk (8) and kgroups (5); 0 = the wave reads them from its
// descriptor (more members, larger shapes, or the switch off).
struct NarrowPre {
    static constexpr int N = 6;
    const void *base = nullptr;
    uint32_t shift = 0;
    uint32_t geo[N] = {0u, 0u, 0u, 0u, 0u, 0u};
};
inline uint32_t narrow_geo(const MfmaTileArgs &a) {
    if (a.tiles == 0u || a.tiles >= 1024u || a.ksteps >= 256u || a.stage_chunk >= 256u ||
        a.kgroups == 0u || a.kgroups >= 32u)
        return 0u;
    return a.tiles | ((a.red_local ? 1u : 0u) << 10) | (a.ksteps << 11) | (a.stage_chunk << 19) |
           (a.kgroups << 27);
}
// Work items of a narrow wave in launch order (XCD-local waves: whole groups of 8 tiles).
__host__ __device__ inline uint32_t narrow_items(uint32_t tiles, uint32_t kgroups, bool local) {
    return (local ? (tiles + 7u) / 8u * 8u : tiles) * kgroups;
}

// Per-wave shares of the 8 XCDs (xcd_order 2), host and device.  Workgroup b runs on XCD
// x = b % 8 as that XCD's s-th workgroup, s = b / 8.  Every wave w of the group (items
// [start[w], start[w+1]), cnt = 8q + r) gives each XCD a contiguous share of its items: q, plus
// one of the r leftover items for r XCDs taken cyclically where the previous wave's leftovers
// stopped (so every XCD gets exactly as many items as workgroups).  XCD x runs its shares in
// wave order, so waves placed first (the host sorts a group's waves by stages per item,
// descending) start first on every XCD.  Returns the item and sets w; a bijection of [0, n).
__host__ __device__ __forceinline__ uint32_t balanced_item(uint32_t b, const uint32_t *start,
                                                           uint32_t nw, uint32_t &w) {
    const uint32_t x = b & 7u;
    uint32_t s = b >> 3, off = 0;
    for (w = 0; w + 1u < nw; ++w) {
        const uint32_t cnt = start[w + 1u] - start[w], q = cnt >> 3, r = cnt & 7u;
        const uint32_t here = q + (((x - off) & 7u) < r ? 1u : 0u);
        if (s < here) break;
        s -= here;
        off = (off + r) & 7u;
    }
    const uint32_t cnt = start[w + 1u] - start[w], q = cnt >> 3, r = cnt & 7u;
    const uint32_t ring = ((1u << r) - 1u) << off;
    const uint32_t extra = (ring | (ring >> 8)) & 0xffu & ((1u << x) - 1u);  // XCDs y < x
    return start[w] + x * q + (uint32_t)__builtin_popcount(extra) + s;
}

// Work item of this workgroup and its wave.  Workgroups are handed to the 8 XCDs round-robin
// (workgroup b runs on XCD b % 8), each XCD with its own L2.  xcd_order 1: XCD x runs the
// contiguous item range [x*q + min(x, r), ...) (n = 8q + r items): consecutive tiles of one
// token tile, whose gathers read the token tile's input rows, share that XCD's L2 instead of
// every XCD fetching every token tile.  xcd_order 2: per-wave shares (balanced_item), which keep
// that locality and also spread long and short waves evenly over the XCDs.
__device__ __forceinline__ uint32_t group_item_wave(const MfmaGroup &g, uint32_t &w) {
    const uint32_t b = blockIdx.x;
    if (g.xcd_order == 2u) return balanced_item(b, g.start, g.n, w);
    uint32_t item = b;
    if (g.xcd_order) {
        const uint32_t n = gridDim.x, x = b & 7u, s = b >> 3, q = n >> 3, r = n & 7u;
        item = x * q + min(x, r) + s;
    }
    w = 0;
    while (w + 1u < g.n && item >= g.start[w + 1u]) ++w;
    return item;
}

// Epilogue of a 64-token-per-wave MFMA tile: lane holds C[4g + i][lane & 15] of every 16x16
// accumulator tile.  Split-K stores the fp32 partial; otherwise bias, activation ACT, residual /
// cout_map and the fp16 (RNE) store, 2 bytes per lane per access.
template <int NT, int ACT>
__device__ __forceinline__ void mfma_epilogue_direct(const MfmaTileArgs &a,
                                                     const f4_t (&acc)[NT / 16][4], uint32_t tile,
                                                     uint32_t tok0, uint32_t zgroup, int lane,
                                                     int wave) {
    constexpr int NB = NT / 16;
    const int g = lane >> 4;
    const uint32_t n_base = tile * (uint32_t)NT + 4u * (uint32_t)g;
    const uint32_t t_base = tok0 + (uint32_t)wave * 64u + (uint32_t)(lane & 15);
    if (a.part) {  // split-K: fp32 partial tile, epilogue in k44_splitk_epilogue_kernel
        float *pz = a.part + (uint64_t)zgroup * a.cout * a.tokens;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t j = n_base + 16u * nb + (uint32_t)i;
#pragma unroll
                for (int tb = 0; tb < 4; ++tb)
                    pz[(uint64_t)j * a.tokens + t_base + 16u * tb] = acc[nb][tb][i];
            }
        return;
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t j = n_base + 16u * nb + (uint32_t)i;
            const float b = a.bias ? __half2float(a.bias[j]) : 0.0f;
            const uint64_t oj = a.cmap ? (uint64_t)a.cmap[j] : (uint64_t)j;
            if (a.cmap && oj == K44_CMAP_EMPTY) continue;  // empty slot of a pattern-sorted tile
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
                if (!tok_stored(a, t_base + 16u * tb)) continue;  // halo column of a plane row
                const uint64_t o = oj * a.out_stride + tok_y(a, t_base + 16u * tb);
                const float r = a.R ? __half2float(a.R[o]) : 0.0f;
                const float v = acc[nb][tb][i] + b;
                const float y = a.cmap ? act_c<ACT>(v + r) : act_c<ACT>(v) + r;
                a.Y[o] = __float2half_rn(y);
            }
        }
}

// LDS floats one wave needs for mfma_epilogue_lds (16 neurons x 64 tokens, padded rows).
constexpr int EPI_PITCH = 68;
constexpr int EPI_WAVE_FLOATS = 16 * EPI_PITCH;

// The same epilogue with the accumulators transposed through LDS, for waves whose output and
// residual offsets are multiples of 8 elements (MfmaTileArgs::epi_vec).  Each wave writes its
// accumulators, 16 neurons at a time, to its own LDS region `ws` ([neuron][64 tokens],
// EPI_WAVE_FLOATS floats) and reads them back as 8 consecutive tokens of one neuron per lane:
// 16-byte residual loads and 16-byte stores, 8 lanes covering a neuron's 64 tokens (split-K
// partials: two 16-byte stores).  Bias and, without a cout_map, the activation are applied
// before the transpose, the rest after it: the same operations in the same order as
// mfma_epilogue_direct, so the same results.
// Memory accesses go through the global address space (the descriptor's pointers would
// otherwise compile to flat accesses, which also count on the LDS counter: every LDS wait of the
// transpose would wait for the stores before it).  The cout_map entries of all blocks load in
// one batch up front, each block's biases and residual rows together before its transpose (null
// tables stood in for by the weights or the output, unused).
template <int NT, int ACT>
__device__ __forceinline__ void mfma_epilogue_lds(const MfmaTileArgs &a,
                                                  const f4_t (&acc)[NT / 16][4], uint32_t tile,
                                                  uint32_t tok0, uint32_t zgroup, int lane,
                                                  int wave, float *ws) {
    typedef const __attribute__((address_space(1))) uint16_t gu16;
    typedef const __attribute__((address_space(1))) gd_u2 gu2;
    typedef const __attribute__((address_space(1))) u4_t gu4;
    typedef __attribute__((address_space(1))) u4_t gu4w;
    typedef __attribute__((address_space(1))) f4_t gf4w;
    constexpr int NB = NT / 16;
    const int g = lane >> 4, c = lane & 15;
    const bool split = a.part != nullptr, mapped = a.cmap != nullptr;
    const uint32_t t_wave = tok0 + (uint32_t)wave * 64u;
    const int ch = lane & 7;  // read side: 8-token chunk of the lane
    const uint32_t t = t_wave + 8u * (uint32_t)ch;
    const uint32_t j_tile = tile * (uint32_t)NT;
    // cout_map entries of the read side (neurons 8q + lane / 8 of each block), all blocks
    uint32_t cb[NB][2];
    {
        gu16 *cm = (gu16 *)(mapped ? (const void *)a.cmap : (const void *)a.Wf);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int q = 0; q < 2; ++q)
                cb[nb][q] = cm[j_tile + 16u * nb + 8u * q + (uint32_t)(lane >> 3)];
    }
    const uint16_t *bsrc = (const uint16_t *)(a.bias ? (const void *)a.bias : (const void *)a.Wf);
    const uint64_t ty = split ? 0u : tok_y(a, t);
    // output offset of read-side row q of block nb, ~0 for an empty slot of a pattern-sorted tile
    auto out_off = [&](int nb, int q) -> uint64_t {
        const uint32_t j = j_tile + 16u * nb + 8u * q + (uint32_t)(lane >> 3);
        const uint64_t oj = mapped ? (uint64_t)cb[nb][q] : (uint64_t)j;
        return (mapped && oj == K44_CMAP_EMPTY) ? ~0ull : oj * a.out_stride + ty;
    };
    const __half *rbase = a.R ? a.R : a.Y;  // without a residual: the output stands in (unused)
    auto res_load = [&](int nb, u4_t (&r)[2]) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const uint64_t o = out_off(nb, q);
            r[q] = *(gu4 *)(rbase + (o == ~0ull ? 0u : o));
        }
    };
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        // this block's biases (neurons 4g .. 4g+3: one 8-byte load) and residual rows, together
        const gd_u2 bb = *(gu2 *)(bsrc + j_tile + 16u * nb + 4u * (uint32_t)g);
        u4_t rcur[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
        if (!split && a.R) res_load(nb, rcur);  // in flight during the transpose
        // write: lane holds neurons 4g..4g+3 of block nb, tokens 16 tb + c
        const __half *bh = reinterpret_cast<const __half *>(&bb);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float b = (!split && a.bias) ? __half2float(bh[i]) : 0.0f;
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
                float v = acc[nb][tb][i];
                if (!split) {
                    v = v + b;
                    if (!mapped) v = act_c<ACT>(v);
                }
                ws[(4 * g + i) * EPI_PITCH + 16 * tb + c] = v;
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        // read: neuron n = 8q + lane / 8 of the block, tokens 8 ch .. 8 ch + 7
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int n = 8 * q + (lane >> 3);
            const f4_t v0 = *reinterpret_cast<const f4_t *>(&ws[n * EPI_PITCH + 8 * ch]);
            const f4_t v1 = *reinterpret_cast<const f4_t *>(&ws[n * EPI_PITCH + 8 * ch + 4]);
            if (split) {
                const uint32_t j = j_tile + 16u * nb + (uint32_t)n;
                gf4w *pz = (gf4w *)(a.part + ((uint64_t)zgroup * a.cout + j) * a.tokens + t);
                pz[0] = v0;
                pz[1] = v1;
                continue;
            }
            const uint64_t o = out_off(nb, q);
            if (o == ~0ull) continue;  // empty slot of a pattern-sorted tile
            const float vv[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
            const __half *rh = reinterpret_cast<const __half *>(&rcur[q]);
            u4_t out;
            __half *oh = reinterpret_cast<__half *>(&out);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float r = a.R ? __half2float(rh[k]) : 0.0f;
                const float y = mapped ? act_c<ACT>(vv[k] + r) : vv[k] + r;
                oh[k] = __float2half_rn(y);
            }
            *(gu4w *)(a.Y + o) = out;
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
}

// Epilogue of the wide MFMA kernels, one activation instance per wave (the unrolled epilogue
// with the whole activation switch inlined per element outgrows the instruction cache).  With
// a.epi_vec the LDS-transposed form: `ws` is this wave's region of EPI_WAVE_FLOATS floats, and
// every wave of the workgroup must be done with the LDS it overlays.
template <int NT>
__device__ __forceinline__ void mfma_tile_epilogue(const MfmaTileArgs &a,
                                                   const f4_t (&acc)[NT / 16][4], uint32_t tile,
                                                   uint32_t tok0, uint32_t zgroup, int lane,
                                                   int wave, float *ws) {
    if (a.epi_vec) {
        K44_WITH_ACT(a.act, mfma_epilogue_lds<NT, A_>(a, acc, tile, tok0, zgroup, lane, wave, ws))
    } else {
        K44_WITH_ACT(a.act, mfma_epilogue_direct<NT, A_>(a, acc, tile, tok0, zgroup, lane, wave))
    }
}

// MIS: segment rows may start at any element (token-shifted taps, single-frame 2-D planes):
// each lane loads the two aligned 16-byte chunks around its 8 tokens and shifts them into
// place (shift_elems) before the LDS store; needs 32-row stages.
template <int NT, int MT, int ROWS, bool MIS = false>
__global__ __launch_bounds__(MT) void k44_mfma_tile_kernel(K44_GROUP_PARAMS) {
    static_assert(!MIS || ROWS == 32, "misaligned rows: 32-row stages");
    K44_GROUP_BIND;
    uint32_t w;
    const uint32_t item = group_item_wave(grp, w);
    const MfmaTileArgs a = grp.waves[w];
    const uint32_t local = item - grp.start[w];
    const uint32_t tile = local % a.tiles, rest = local / a.tiles;
    const uint32_t ytile = rest % a.ttiles, zgroup = rest / a.ttiles;
    constexpr int NB = NT / 16;              // 16-neuron blocks per tile
    constexpr int PITCH = MT + 16;           // LDS row pitch in halves (32-byte skew)
    constexpr int CPR = MT / 8;              // 16-byte chunks per position row
    constexpr int CPT = ROWS * CPR / MT;     // chunks per thread per stage (= ROWS / 8)
    __shared__ __attribute__((aligned(16))) _Float16 lds[2][ROWS][PITCH];
    static_assert(sizeof(lds) >= (MT / 64) * EPI_WAVE_FLOATS * sizeof(float), "epilogue LDS");

    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t tok0 = ytile * (uint32_t)MT;
    const uint64_t *segr = a.seg + (uint64_t)tile * a.K;
    const uint32_t stages = a.K * a.S / (uint32_t)ROWS;
    const uint32_t st_begin = zgroup * a.stage_chunk;
    const uint32_t st_end = min(stages, st_begin + a.stage_chunk);

    f4_t acc[NB][4];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) acc[nb][tb] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int g = lane >> 4;
    const int tr_row = 8 * g + ((lane & 15) >> 2);  // row read by this lane (first half)
    const int tr_col = wave * 64 + 4 * (lane & 3);  // token column (+16 per token block)
    constexpr int SUBS = ROWS / 32;                  // 32-deep MFMA K-steps per stage
    const h8_t *wf = reinterpret_cast<const h8_t *>(a.Wf) +
                     (uint64_t)tile * a.ksteps * NB * 64 + lane;

    // Stage st covers index-row positions [st*ROWS, st*ROWS + ROWS) — inside one segment.
    // Thread chunk i of a stage: row (tid + i*MT) / CPR, tokens ((tid + i*MT) % CPR) * 8 .. +8,
    // at canvas offset xo[i] of the segment row (the same for every stage).
    uint64_t xo[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) xo[i] = tok_x(a, tok0 + ((tid + i * MT) % CPR) * 8u);
    u4_t xr[CPT];  // X of the next stage, in flight during the current stage's MFMAs
    u4_t xh[MIS ? CPT : 1];        // MIS: the aligned chunk after xr's
    uint32_t xm[MIS ? CPT : 1];    // MIS: element offset of the lane's tokens in xr:xh
    h8_t wn[SUBS][NB], wc[SUBS][NB];  // A fragments: next stage (in flight), current stage
    auto load_x = [&](uint32_t st) {
        const uint32_t kk = st * (uint32_t)ROWS;
        const uint32_t k = kk / a.S, s0 = kk - k * a.S;
        const uint64_t e0 = segr[k] + (uint64_t)s0 * a.step;
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = tid + i * MT;
            const uint64_t e = e0 + (uint64_t)(c / CPR) * a.step + xo[i];
            if constexpr (MIS) {
                const __half *p = a.X + (e & ~7ull);
                xr[i] = *reinterpret_cast<const u4_t *>(p);
                xh[i] = *reinterpret_cast<const u4_t *>(p + 8);
                xm[i] = (uint32_t)(e & 7u);
            } else {
                xr[i] = *reinterpret_cast<const u4_t *>(a.X + e);
            }
        }
    };
    auto store_x = [&](int buf) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = tid + i * MT;
            u4_t v = xr[i];
            if constexpr (MIS) v = shift_elems(xr[i], xh[i], xm[i]);
            *reinterpret_cast<u4_t *>(&lds[buf][c / CPR][(c % CPR) * 8]) = v;
        }
    };
    {
        load_x(st_begin);
#pragma unroll
        for (int u = 0; u < SUBS; ++u)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                wc[u][nb] = wf[((uint64_t)(st_begin * SUBS + u) * NB + nb) * 64];
        store_x(0);
    }
    __syncthreads();

    for (uint32_t st = st_begin; st < st_end; ++st) {
        const int buf = (int)((st - st_begin) & 1u);
        const bool more = st + 1 < st_end;
        if (more) {  // issue next stage's X and W loads; consumed only after this stage's math
            load_x(st + 1);
#pragma unroll
            for (int u = 0; u < SUBS; ++u)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    wn[u][nb] = wf[((uint64_t)((st + 1) * SUBS + u) * NB + nb) * 64];
        }
#pragma unroll
        for (int u = 0; u < SUBS; ++u) {
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
                const _Float16 *p = &lds[buf][u * 32 + tr_row][tr_col + 16 * tb];
                const h4_t lo = lds_read_tr16(p);
                const h4_t hi = lds_read_tr16(p + 4 * PITCH);
                const h8_t b = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    acc[nb][tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wc[u][nb], b,
                                                                         acc[nb][tb], 0, 0, 0);
            }
        }
        if (more) {
            store_x(buf ^ 1);
#pragma unroll
            for (int u = 0; u < SUBS; ++u)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) wc[u][nb] = wn[u][nb];
        }
        __syncthreads();
    }

    // The last stage ended with a barrier after its LDS reads: the LDS is free for the epilogue.
    mfma_tile_epilogue<NT>(a, acc, tile, tok0, zgroup, lane, wave,
                           reinterpret_cast<float *>(&lds[0][0][0]) + wave * EPI_WAVE_FLOATS);
}

}  // namespace k44dev
