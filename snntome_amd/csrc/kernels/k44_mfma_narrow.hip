// Translation unit of the narrow MFMA kernel: dense-cluster waves over at most 16 tokens
// (decode steps).  The wide tile kernel (k44_mfma_tile.hpp) gives every wave 64 tokens; at 16
// real tokens three quarters of its work and of its split-K partials would be padding, and the
// wave is bound by streaming its weights once.  Here:
//  * one workgroup (4 waves) = one NT-neuron tile x one chunk of the contraction (a range of
//    32-deep k-steps) x 16 tokens;
//  * the chunk's X rows (16 tokens = 32 bytes each) are gathered once into LDS, row-major; the
//    B operand comes from ds_read_b64_tr_b16 exactly as in the wide kernel (lane 16g+4j+m reads
//    row 8g+j (+4), tokens 4m..4m+3);
//  * each wave owns 16-neuron blocks (NT = 64: one each; NT = 128: two) or, for NT < 64, the
//    waves of a block take its k-steps round-robin and meet in LDS in a fixed order;
//  * A fragments (host-arranged [tile][k-step][16-block][lane][8]) stream from HBM with 8 k-steps
//    of loads in flight per wave before the first MFMA that needs them;
//  * one chunk: fused epilogue; several: fp32 partials, summed in chunk order (bit-
//    reproducible) by the last workgroup of the tile to arrive (64 / 128-neuron tiles in
//    whole-plan runs, narrow_reduce_last) or by k44_splitk_epilogue_kernel.  The in-launch
//    reduction publishes its partials as device-coherent stores instead of through a release
//    fence: an agent-scope release is an L2 write-back on this GPU (an earlier design with one
//    per workgroup measured 4x slower on decode-sized waves).
// Columns 16..stride-1 of the output rows are not written.
#include "k44_launch.hpp"
#include "k44_sumsq.hpp"

namespace k44dev {

constexpr int NARROW_MAX_ROWS = 512;  // rows of one chunk held in LDS
constexpr int NARROW_PITCH = 24;      // halves per LDS row (16 tokens + 8 skew)
typedef float f2_t __attribute__((ext_vector_type(2)));

// Fused epilogue of a whole-contraction chunk: lane holds C[4g + i][t] of BPW 16-neuron blocks,
// neuron j = j0[bi] + i.  The cout_map entries and biases of all 4 * BPW outputs are loaded in
// one batch, then the residuals they address in a second, all through the global address space
// (pointers read from the descriptor would compile to flat accesses, and a load per output under
// the branch for empty slots makes the compiler wait for each in turn).  Null tables are stood
// in for by buffers the index is valid in (weights for cout_map / bias, the output for the
// residual), their values unused.  Arithmetic as in k44_splitk_epilogue_kernel.
// narrow_epi_load issues the loads (split-K waves issue them before their reduction, so they
// complete under it), narrow_epi_store forms and stores the outputs.
template <int BPW>
struct NarrowEpi {
    uint32_t bb[BPW][4], rb[BPW][4];
    uint64_t o[BPW][4];  // output element, ~0 for an empty cout_map slot
};

// The two batches separately: cout_map entries and biases (narrow_epi_maps), then the
// residuals at the output rows they name (narrow_epi_res).  The long kernel issues the first
// with its first X gather and the second once that gather has arrived, so neither round trip
// follows the contraction.
template <int BPW>
__device__ __forceinline__ void narrow_epi_maps(const MfmaTileArgs &a, const uint32_t (&j0)[BPW],
                                                uint32_t (&cb)[BPW][4], NarrowEpi<BPW> &e) {
    typedef const __attribute__((address_space(1))) uint16_t gu16;
    gu16 *cm = (gu16 *)(a.cmap ? (const void *)a.cmap : (const void *)a.Wf);
    gu16 *bs = (gu16 *)(a.bias ? (const void *)a.bias : (const void *)a.Wf);
#pragma unroll
    for (int bi = 0; bi < BPW; ++bi)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            cb[bi][i] = cm[j0[bi] + (uint32_t)i];
            e.bb[bi][i] = bs[j0[bi] + (uint32_t)i];
        }
}

template <int BPW>
__device__ __forceinline__ void narrow_epi_res(const MfmaTileArgs &a, const uint32_t (&j0)[BPW],
                                               uint32_t t, const uint32_t (&cb)[BPW][4],
                                               NarrowEpi<BPW> &e) {
    typedef const __attribute__((address_space(1))) uint16_t gu16;
    gu16 *rs = (gu16 *)(a.R ? (const void *)a.R : (const void *)a.Y);
#pragma unroll
    for (int bi = 0; bi < BPW; ++bi)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint64_t oj = a.cmap ? (uint64_t)cb[bi][i] : (uint64_t)(j0[bi] + (uint32_t)i);
            e.o[bi][i] = (a.cmap && oj == K44_CMAP_EMPTY) ? ~0ull : oj * a.out_stride + t;
            e.rb[bi][i] = rs[e.o[bi][i] == ~0ull ? (uint64_t)t : e.o[bi][i]];
        }
}

template <int BPW>
__device__ __forceinline__ void narrow_epi_load(const MfmaTileArgs &a, const uint32_t (&j0)[BPW],
                                                uint32_t t, NarrowEpi<BPW> &e) {
    uint32_t cb[BPW][4];
    narrow_epi_maps<BPW>(a, j0, cb, e);
    narrow_epi_res<BPW>(a, j0, t, cb, e);
}

template <int BPW>
__device__ __forceinline__ void narrow_epi_store(const MfmaTileArgs &a, const f4_t (&acc)[BPW],
                                                 const NarrowEpi<BPW> &e, uint16_t (&out)[BPW][4]) {
    typedef __attribute__((address_space(1))) uint16_t gu16w;
    // every value formed before the first store (a store between a residual load and its use
    // would be waited for with it: both count on the same counter)
#pragma unroll
    for (int bi = 0; bi < BPW; ++bi)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float b = a.bias ? __half2float(__ushort_as_half((unsigned short)e.bb[bi][i])) : 0.0f;
            const float r = a.R ? __half2float(__ushort_as_half((unsigned short)e.rb[bi][i])) : 0.0f;
            const float v = acc[bi][i] + b;
            out[bi][i] = __half_as_ushort(
                __float2half_rn(a.cmap ? apply_act(v + r, a.act) : apply_act(v, a.act) + r));
        }
#pragma unroll
    for (int bi = 0; bi < BPW; ++bi)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (e.o[bi][i] != ~0ull) ((gu16w *)a.Y)[e.o[bi][i]] = out[bi][i];  // not an empty slot
}

template <int BPW>
__device__ __forceinline__ void narrow_fused_epilogue(const MfmaTileArgs &a, const f4_t (&acc)[BPW],
                                                      const uint32_t (&j0)[BPW], uint32_t t) {
    NarrowEpi<BPW> e;
    uint16_t out[BPW][4];
    narrow_epi_load<BPW>(a, j0, t, e);
    narrow_epi_store<BPW>(a, acc, e, out);
}

// Producer side of a folded RMSNorm (a.norm_part set): the tile's stored fp16 outputs (lane
// (g, t): out[bi][i] of channel slot j0[bi] + i, token t) summed squared per token, exactly:
// over the lanes of one token (xor 16, 32), then the 4 waves in LDS; wave 0 stores the tile's
// slot (16 tokens x 2 words).  The readers of the norm, in later launches, add every slot
// themselves (rms_inv_from_slots).  Every wave of the workgroup calls this (one barrier).
template <int BPW>
__device__ __forceinline__ void narrow_norm_publish(const MfmaTileArgs &a, const NarrowEpi<BPW> &e,
                                                    const uint16_t (&out)[BPW][4],
                                                    uint32_t tile) {
    typedef unsigned long long u64;
    typedef __attribute__((address_space(1))) u64 gu64;
    __shared__ SumSq red[4][16];
    SumSq s = sumsq_zero();
#pragma unroll
    for (int bi = 0; bi < BPW; ++bi)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (e.o[bi][i] != ~0ull) sumsq_add(s, out[bi][i]);  // empty slots store nothing
    s = sumsq_wave_reduce(s, 16);
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    if (lane < 16u) red[wave][lane] = s;
    __syncthreads();
    if (wave != 0u || lane >= 16u) return;
    SumSq q = red[0][lane];
    sumsq_merge(q, red[1][lane]);
    sumsq_merge(q, red[2][lane]);
    sumsq_merge(q, red[3][lane]);
    q = sumsq_norm(q);  // one tile: the top limb and the flags fit 32 bits each
    gu64 *slot = (gu64 *)(a.norm_part + ((uint64_t)tile * 16u + lane) * 4u);
    slot[0] = (u64)q.l0 | (q.l1 << 32);
    slot[1] = (u64)(uint32_t)q.l2 | ((u64)q.sp << 32);
}

// Split-K reduced inside the launch (a.arrive set; 64 / 128-neuron tiles).  Every workgroup of
// a tile stores its chunk's partial, then counts itself in at the tile's arrival counter; the
// workgroup that arrives last sums the kgroups partials in chunk order (the order of
// k44_splitk_epilogue_kernel, so the outputs are the same bits) and runs the fused epilogue.
// Visibility without an L2 write-back: the partials are stored and read as agent-scope relaxed
// atomics (stores and loads marked device-coherent: the other XCDs' L2 caches are not
// consulted), each wave waits for its stores to complete (vmcnt 0) before the barrier that
// precedes the counter increment, and the last workgroup reads only after the increment has
// returned.  An agent-scope release fence would instead write back the whole L2 of the XCD.
// The last workgroup resets the counter to zero for the next launch (no clearing kernel or
// memset, so HIP-graph replays need no extra node).  Lane (g, t) holds C[4g + i][t] of BPW
// 16-neuron blocks; its 4 values of block bi are contiguous in the partial layout
// [z][cout/4][16][4]: index ((z * cout + j0) * 16 + 4 t + i).
// XCD-local form (a.red_local): the same steps through the L2 of the one XCD every chunk of
// the tile runs on: plain stores (written through L1 into L2), an L2 atomic for the counter
// and loads that miss in L1 (sc0); no access leaves the XCD.  (Were the chunks ever placed on
// different XCDs, no workgroup would count last and the tile's counter would stay nonzero:
// the host checks the counters after each run.)
template <int BPW>
__device__ __forceinline__ bool narrow_reduce_last(const MfmaTileArgs &a, f4_t (&acc)[BPW],
                                                   const uint32_t (&j0)[BPW], uint32_t t,
                                                   uint32_t tile, uint32_t z) {
    typedef unsigned long long u64;
    typedef __attribute__((address_space(1))) u64 gu64;
    typedef __attribute__((address_space(1))) uint32_t gu32;
    __shared__ uint32_t last;
    const bool xl = a.red_local != 0u;
    gu64 *pp = (gu64 *)(a.part);
    // (XCD-local counters one 128-byte line apart: tiles of one line run on different XCDs)
    gu32 *cnt = (gu32 *)(a.arrive) + tile * (xl ? 32u : 1u);
    auto slot = [&](uint32_t zz, int bi) -> uint64_t {
        return (((uint64_t)zz * a.cout + j0[bi]) * 16u + 4u * t) >> 1;
    };
#pragma unroll
    for (int bi = 0; bi < BPW; ++bi) {
        const uint64_t s = slot(z, bi);
        const u64 v0 = __builtin_bit_cast(u64, __builtin_shufflevector(acc[bi], acc[bi], 0, 1));
        const u64 v1 = __builtin_bit_cast(u64, __builtin_shufflevector(acc[bi], acc[bi], 2, 3));
        if (xl) {
            pp[s] = v0;
            pp[s + 1] = v1;
        } else {
            __hip_atomic_store(pp + s, v0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(pp + s + 1, v1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's partial stores performed
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t before;
        if (xl) {
            before = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        } else {
            before = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        last = before == a.kgroups - 1u;
    }
    __syncthreads();
    if (!last) return false;
    const uint32_t kg = a.kgroups;
    // (XCD-local: byte offsets from the partial buffer, below 2 GiB by the host's check)
    const __amdgpu_buffer_rsrc_t prs =
        __builtin_amdgcn_make_buffer_rsrc(a.part, (short)0, 0x7fffffff, 0x00020000);
    f4_t sum[BPW];
    constexpr uint32_t ZB = 8u;  // planes loaded together
    for (uint32_t z0 = 0; z0 < kg; z0 += ZB) {
        u64 lo[ZB][BPW], hi[ZB][BPW];
#pragma unroll
        for (uint32_t u = 0; u < ZB; ++u) {
            const uint32_t zz = min(z0 + u, kg - 1u);
#pragma unroll
            for (int bi = 0; bi < BPW; ++bi) {
                const uint64_t s = slot(zz, bi);
                if (xl) {
                    const uint32_t off = (uint32_t)(s * 8u);
                    lo[u][bi] = __builtin_bit_cast(u64, __builtin_amdgcn_raw_buffer_load_b64(prs, off, 0, 1));
                    hi[u][bi] = __builtin_bit_cast(u64, __builtin_amdgcn_raw_buffer_load_b64(prs, off + 8u, 0, 1));
                } else {
                    lo[u][bi] = __hip_atomic_load(pp + s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    hi[u][bi] = __hip_atomic_load(pp + s + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
#pragma unroll
        for (uint32_t u = 0; u < ZB; ++u) {
            const uint32_t zz = z0 + u;
            if (zz < kg) {
#pragma unroll
                for (int bi = 0; bi < BPW; ++bi) {
                    // this workgroup's own chunk from its registers (the same bits it stored)
                    const f4_t p = zz == z ? acc[bi]
                                           : __builtin_shufflevector(
                                                 __builtin_bit_cast(f2_t, lo[u][bi]),
                                                 __builtin_bit_cast(f2_t, hi[u][bi]), 0, 1, 2, 3);
                    if (zz == 0u) {
                        sum[bi] = p;
                    } else {
                        sum[bi][0] += p[0];
                        sum[bi][1] += p[1];
                        sum[bi][2] += p[2];
                        sum[bi][3] += p[3];
                    }
                }
            }
        }
    }
#pragma unroll
    for (int bi = 0; bi < BPW; ++bi) acc[bi] = sum[bi];
    // every workgroup of the tile has arrived: the counter is zero again for the next launch
    if (threadIdx.x == 0) {
        if (xl)
            __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        else
            __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return true;
}

template <int NT>
__global__ __launch_bounds__(256) void k44_mfma_narrow_kernel(K44_GROUP_PARAMS) {
    K44_GROUP_BIND;
    constexpr int NB = NT / 16;                // 16-neuron blocks per tile
    constexpr int BL = NB < 4 ? NB : 4;        // distinct blocks handled at once by the 4 waves
    constexpr int KW = 4 / BL;                 // waves sharing a block (split k-steps)
    constexpr int BPW = NB / BL;               // blocks per wave
    constexpr int AB = 16;                     // k-steps of A fragments in flight per wave
    __shared__ __attribute__((aligned(16))) _Float16 xl[NARROW_MAX_ROWS][NARROW_PITCH];
    __shared__ f4_t red[KW > 1 ? 4 : 1][64];

    uint32_t w = 0;
    while (w + 1u < grp.n && blockIdx.x >= grp.start[w + 1u]) ++w;
    const MfmaTileArgs a = grp.waves[w];
    const uint32_t local = blockIdx.x - grp.start[w];
    const uint32_t tile = local % a.tiles, zgroup = local / a.tiles;
    const uint32_t ks_begin = zgroup * a.stage_chunk;
    const uint32_t ks_end = min(a.ksteps, ks_begin + a.stage_chunk);
    const uint32_t r0 = ks_begin * 32u, nrows = (ks_end - ks_begin) * 32u;

    const int tid = (int)threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
    // Segment starts are read-only: scalar loads through the constant address space (they wait
    // on the scalar counter only, not on the A-fragment loads already in flight).
    const kconst_u64 *segr = (const kconst_u64 *)(a.seg) + (uint64_t)tile * a.K;
    const int blk0 = wave % BL, kw = wave / BL;
    const h8_t *wf = reinterpret_cast<const h8_t *>(a.Wf) + (uint64_t)tile * a.ksteps * NB * 64 +
                     lane;

    // The first AB k-steps' A fragments are requested before the X gather, so both are in
    // flight together (a chunk is a handful of k-steps: the workgroup is latency-bound).  Loads
    // past the chunk re-read its last k-step (unused): a fixed load count per wave lets every
    // later wait be partial.
    h8_t af[AB][BPW];
#pragma unroll
    for (int u = 0; u < AB; ++u) {
        const uint32_t k2 = min(ks_begin + (uint32_t)kw + (uint32_t)u * KW, ks_end - 1u);
#pragma unroll
        for (int i = 0; i < BPW; ++i)
            af[u][i] = __builtin_nontemporal_load((const __attribute__((address_space(1))) h8_t *)(
                wf + ((uint64_t)k2 * NB + blk0 + BL * i) * 64));
    }

    // X rows [r0, r0 + nrows) of the tile's index row, 16 tokens each, into LDS.  Pass q of a
    // wave covers 32 consecutive rows starting at a multiple of 32, i.e. inside one segment
    // (S % 32 == 0): its segment start is wave-uniform.  All loads are issued before the first
    // LDS store.
    constexpr int XQ = NARROW_MAX_ROWS * 2 / 256;  // 16-byte chunks per thread at most
    u4_t xv[XQ];
    // first row of each pass; passes past the chunk re-read its last 32 rows (unused), so the
    // load count is fixed and the stores below wait only once.  The scalar segment-start loads
    // of all passes are issued together, then all X loads.
    uint64_t sb[XQ];
#pragma unroll
    for (int q = 0; q < XQ; ++q) {
        const uint32_t r = r0 + min((uint32_t)(32 * (wave + 4 * q)), nrows - 32u);
        const uint32_t k = r / a.S;
        sb[q] = segr[k] + (uint64_t)(r - k * a.S) * a.step;
    }
#pragma unroll
    for (int q = 0; q < XQ; ++q)
        xv[q] = *(const __attribute__((address_space(1))) u4_t *)(
            a.X + sb[q] + (uint64_t)(lane >> 1) * a.step + (uint32_t)(lane & 1) * 8u);
#pragma unroll
    for (int q = 0; q < XQ; ++q) {
        const uint32_t rb = (uint32_t)(32 * (wave + 4 * q));
        if (rb < nrows)
            *reinterpret_cast<u4_t *>(&xl[rb + (uint32_t)(lane >> 1)][(lane & 1) * 8]) = xv[q];
    }
    __syncthreads();

    const int g = lane >> 4;
    const int tr_row = 8 * g + ((lane & 15) >> 2);
    const int tr_col = 4 * (lane & 3);
    f4_t acc[BPW];
#pragma unroll
    for (int i = 0; i < BPW; ++i) acc[i] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

    for (uint32_t ks = ks_begin + (uint32_t)kw; ks < ks_end; ks += (uint32_t)AB * KW) {
        if (ks != ks_begin + (uint32_t)kw) {  // later batches (chunks longer than AB k-steps)
#pragma unroll
            for (int u = 0; u < AB; ++u) {
                const uint32_t k2 = min(ks + (uint32_t)u * KW, ks_end - 1u);
#pragma unroll
                for (int i = 0; i < BPW; ++i)
                    af[u][i] = __builtin_nontemporal_load(
                        (const __attribute__((address_space(1))) h8_t *)(
                            wf + ((uint64_t)k2 * NB + blk0 + BL * i) * 64));
            }
        }
#pragma unroll
        for (int u = 0; u < AB; ++u) {
            const uint32_t k2 = ks + (uint32_t)u * KW;
            if (k2 < ks_end) {
                const _Float16 *p = &xl[(k2 - ks_begin) * 32u + tr_row][tr_col];
                const h4_t lo = lds_read_tr16(p);
                const h4_t hi = lds_read_tr16(p + 4 * NARROW_PITCH);
                const h8_t b = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
                for (int i = 0; i < BPW; ++i)
                    acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[u][i], b, acc[i], 0, 0, 0);
            }
        }
    }

    bool writer = true;  // this wave holds the final (summed over its KW group) accumulators
    if constexpr (KW > 1) {  // waves kw = 0..KW-1 of a block: summed in kw order by wave kw = 0
        red[wave][lane] = acc[0];
        __syncthreads();
        writer = kw == 0;
        if (writer) {
            f4_t s = red[blk0][lane];
            for (int k2 = 1; k2 < KW; ++k2) {
                const f4_t o = red[blk0 + BL * k2][lane];
                s[0] += o[0];
                s[1] += o[1];
                s[2] += o[2];
                s[3] += o[3];
            }
            acc[0] = s;
        }
    }

    // Lane holds C[4g + i][lane & 15]: neuron 16*blk + 4g + i, token lane & 15.
    const uint32_t t = (uint32_t)(lane & 15);
    if (!a.part) {  // whole contraction in this workgroup: fused epilogue
        if (!writer) return;
        uint32_t j0[BPW];
#pragma unroll
        for (int bi = 0; bi < BPW; ++bi)
            j0[bi] = tile * (uint32_t)NT + 16u * (uint32_t)(blk0 + BL * bi) + 4u * (uint32_t)g;
        narrow_fused_epilogue<BPW>(a, acc, j0, t);
        return;
    }

    // Split contraction: fp32 partial [z][cout][16] of this chunk.
    if (writer) {
#pragma unroll
        for (int bi = 0; bi < BPW; ++bi) {
            const uint32_t blk = (uint32_t)(blk0 + BL * bi);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t j = tile * (uint32_t)NT + 16u * blk + 4u * (uint32_t)g + (uint32_t)i;
                a.part[((uint64_t)zgroup * a.cout + j) * 16u + t] = acc[bi][i];
            }
        }
    }
}

// Tiles of 64 / 128 neurons (every wave owns whole 16-neuron blocks): contraction chunks of any
// length, taken in sub-chunks of 16 k-steps (512 rows) through two LDS buffers.  While sub-chunk
// s is multiplied, the X rows of s+1 are in flight to registers, and every A fragment consumed
// is replaced by its counterpart of s+1 (the weights stream without a gap).  A chunk that
// covers the whole contraction runs the fused epilogue: waves of up to a few sub-chunks need no
// split-K partials and no second kernel.
// PROD: 0, or the product form every wave of the launch gathers (a.xprod 2 / 3: two or three
// rows multiplied), fixed at compile time.
// BYY: grid (largest wave's workgroups) x (waves): the wave is blockIdx.y, known without a
// lookup in the group's prefix sums; workgroups past a wave's own count exit at once.
// The weights are read through a buffer resource bounded by the workgroup's chunk: every
// MFMA's operand slot is refilled with the fragment one sub-chunk ahead, and refills past the
// chunk are out-of-range loads, which return zeros without a memory access (the load count
// stays fixed, so every wait is partial, and no request past the chunk delays the split-K
// reduction's wait or the workgroup's end).  Measured on config-5 decode: 0.836 -> 0.8225
// ms/step against refills clamped to the chunk's last k-step (re-reads of it); two sub-chunks
// of fragments in flight per wave instead of one: 0.869 ms/step (each wave's first gather then
// waits behind twice the weight bytes).
// nsh = waves | NarrowPre::shift << 8; geo0..5 / wbase: NarrowPre.  The parameters fill the
// 14 SGPRs that gfx950 preloads (the group's XCD order is not used here).
template <int NT, int PROD, bool BYY>
__global__ __launch_bounds__(256) void k44_mfma_narrow_long_kernel(
    const MfmaTileArgs *grp_waves, const uint32_t *grp_start, uint32_t nsh, uint32_t geo0,
    uint32_t geo1, uint32_t geo2, uint32_t geo3, uint32_t geo4, uint32_t geo5,
    const void *wbase) {
    const MfmaGroup grp{grp_waves, grp_start, nsh & 0xffu, 0u};
    constexpr int NB = NT / 16, BPW = NB / 4, SUBK = 16, AF = SUBK;
    static_assert(NT == 64 || NT == 128, "waves own whole 16-neuron blocks");
    __shared__ __attribute__((aligned(16))) _Float16 xl[2][NARROW_MAX_ROWS][NARROW_PITCH];

    uint32_t w = 0, pos;  // the wave, and the workgroup's position among its work items
    if constexpr (BYY) {
        w = blockIdx.y;
        pos = blockIdx.x;
    } else if (grp.n == 1u) {
        pos = blockIdx.x;
    } else {
        while (w + 1u < grp.n && blockIdx.x >= grp.start[w + 1u]) ++w;
        pos = blockIdx.x - grp.start[w];
    }
    // The wave's weights and geometry from the preloaded arguments where the launch gives them:
    // its first weight loads are then issued before the descriptor is read (the scheduling
    // barrier below keeps the descriptor's scalar loads, and their waits, after them).
    const uint32_t geo = w == 0u   ? geo0
                         : w == 1u ? geo1
                         : w == 2u ? geo2
                         : w == 3u ? geo3
                         : w == 4u ? geo4
                         : w == 5u ? geo5
                                   : 0u;
    const int tid = (int)threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    uint32_t tiles, ksteps, chunk, kgroups, tile, zgroup, ks_begin, ks_end, local;
    bool xlocal;
    __amdgpu_buffer_rsrc_t wr;
    // the work item at pos (idle past the wave's own), its dense index local = z * tiles + tile,
    // and the chunk's A fragments [k-step - ks_begin][16-block][lane][8] (1 KiB per k-step and
    // block)
    auto geometry = [&](const void *wbase) {
        if (xlocal) {
            const uint32_t g8 = pos / (8u * kgroups), r = pos - g8 * 8u * kgroups;
            zgroup = r >> 3;
            tile = g8 * 8u + (r & 7u);
            if (tile >= tiles) return false;
        } else {
            if (pos >= tiles * kgroups) return false;
            tile = pos % tiles;
            zgroup = pos / tiles;
        }
        local = zgroup * tiles + tile;
        ks_begin = zgroup * chunk;
        ks_end = min(ksteps, ks_begin + chunk);
        wr = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(reinterpret_cast<const h8_t *>(wbase) +
                     ((uint64_t)tile * ksteps + ks_begin) * NB * 64u),
            (short)0, (int)((ks_end - ks_begin) * (uint32_t)NB * 1024u), 0x00020000);
        return true;
    };
    // k-step kk of the chunk (relative to ks_begin; past the chunk: zeros, no access), read
    // nontemporally (weights are read once per step)
    auto load_a = [&](uint32_t kk, h8_t (&f)[BPW]) {
#pragma unroll
        for (int i = 0; i < BPW; ++i)
            f[i] = __builtin_bit_cast(
                h8_t, __builtin_amdgcn_raw_buffer_load_b128(
                          wr, ((kk * (uint32_t)NB + (uint32_t)(wave + 4 * i)) * 64u + (uint32_t)lane) * 16u,
                          0, 2));
    };
    h8_t af[AF][BPW];
    if (geo != 0u) {
        tiles = geo & 0x3ffu;
        xlocal = ((geo >> 10) & 1u) != 0u;
        ksteps = (geo >> 11) & 0xffu;
        chunk = (geo >> 19) & 0xffu;
        kgroups = geo >> 27;
        if (!geometry(reinterpret_cast<const char *>(wbase) + ((uint64_t)w << (nsh >> 8))))
            return;
#pragma unroll
        for (int u = 0; u < AF; ++u) load_a((uint32_t)u, af[u]);
    }
    __builtin_amdgcn_sched_barrier(0);
    const MfmaTileArgs a = grp.waves[w];
    if (geo == 0u) {
        tiles = a.tiles;
        xlocal = a.red_local != 0u;
        ksteps = a.ksteps;
        chunk = a.stage_chunk;
        kgroups = a.kgroups;
        if (!geometry(a.Wf)) return;
    }
    const uint32_t nsub = (ks_end - ks_begin + SUBK - 1u) / SUBK;
    const kconst_u64 *segr = (const kconst_u64 *)(a.seg) + (uint64_t)tile * a.K;
    typedef const __attribute__((address_space(1))) u4_t gu4_t;

    // X rows of sub-chunk s: wave pass q covers 32 rows starting at a multiple of 32 (one
    // segment, S % 32 == 0: wave-uniform start); passes past the sub-chunk re-read its last
    // 32 rows (fixed load count).
    // Product gathers (a.xprod = 2 / 3) load the same row chunk of two / three tensors and
    // multiply with the rounding of the unfused multiply commands: fp16(A*B), fp16(A*fp16(B*C)).
    constexpr int XQ = NARROW_MAX_ROWS * 2 / 256;
    constexpr uint32_t xprod = (uint32_t)PROD;  // every wave of the launch gathers this form
    // Folded RMSNorm (xprod 4, 5): the lane's 8 tokens' scales, formed from the producers'
    // slots after the first sub-chunk's loads are issued.
    constexpr bool NORM = xprod == 4u || xprod == 5u;
    float xinv[NORM ? 8 : 1];
    // xprod 5: state rows 1 and 2 of each pass (row 0 in xc), and the passes this workgroup
    // stores the shifted state of
    u4_t xs1[XQ], xs2[XQ];
    uint64_t ownb = 0;
    if constexpr (xprod == 5u) ownb = ((const kconst_u64 *)a.own)[local];
    auto gather = [&](uint32_t s, u4_t (&xv)[XQ], u4_t (&xb)[XQ], u4_t (&xc)[XQ]) {
        const uint32_t kb = ks_begin + s * SUBK;
        const uint32_t nrows = (min(ks_end, kb + SUBK) - kb) * 32u;
        uint64_t sb[XQ];
#pragma unroll
        for (int q = 0; q < XQ; ++q) {
            const uint32_t r = kb * 32u + min((uint32_t)(32 * (wave + 4 * q)), nrows - 32u);
            const uint32_t k = r / a.S;
            sb[q] = segr[k] + (uint64_t)(r - k * a.S) * a.step + (uint64_t)(lane >> 1) * a.step +
                    (uint32_t)(lane & 1) * 8u;
        }
        if (NORM) {
            // the norm's input rows and their gammas (xb holds the gamma bits of each pass)
#pragma unroll
            for (int q = 0; q < XQ; ++q) xv[q] = *(gu4_t *)(a.X + (int64_t)sb[q] + a.xd[0]);
            typedef const __attribute__((address_space(1))) uint16_t gu16;
            if (xprod == 4u) {
                gu16 *gm = (gu16 *)(a.xgamma ? (const void *)a.xgamma : (const void *)a.X);
#pragma unroll
                for (int q = 0; q < XQ; ++q) {
                    const uint64_t row = sb[q] - (uint32_t)(lane & 1) * 8u;
                    xb[q][0] = a.xgamma ? (uint32_t)gm[(row - a.xg_base) >> a.xg_shift] : 0x3c00u;
                }
            } else {
                // the channel's mixing weights and gamma (xb[0..2], one 16-byte load), its
                // state rows (xc, xs1, xs2; rows past rf - 2 repeat the last) and the channel
                // itself (xb[3])
                const uint32_t rf = a.rf;
#pragma unroll
                for (int q = 0; q < XQ; ++q) {
                    const uint32_t c =
                        (uint32_t)((sb[q] - (uint32_t)(lane & 1) * 8u - a.xg_base) >> a.xg_shift);
                    xb[q] = *(gu4_t *)(a.mixg + (uint64_t)c * 8u);
                    xb[q][3] = c;
                    const __half *st = a.state + (uint64_t)c * (rf - 1u) * 16u +
                                       (uint32_t)(lane & 1) * 8u;
                    xc[q] = *(gu4_t *)st;
                    xs1[q] = *(gu4_t *)(st + min(1u, rf - 2u) * 16u);
                    xs2[q] = *(gu4_t *)(st + min(2u, rf - 2u) * 16u);
                }
            }
        } else if (xprod == 0u) {
#pragma unroll
            for (int q = 0; q < XQ; ++q) xv[q] = *(gu4_t *)(a.X + sb[q]);
        } else {
#pragma unroll
            for (int q = 0; q < XQ; ++q) {
                xv[q] = *(gu4_t *)(a.X + (int64_t)sb[q] + a.xd[0]);
                xb[q] = *(gu4_t *)(a.X + (int64_t)sb[q] + a.xd[1]);
            }
            if (xprod == 3u) {
#pragma unroll
                for (int q = 0; q < XQ; ++q) xc[q] = *(gu4_t *)(a.X + (int64_t)sb[q] + a.xd[2]);
            }
        }
    };
    auto store = [&](uint32_t s, int buf, u4_t (&xv)[XQ], const u4_t (&xb)[XQ],
                     const u4_t (&xc)[XQ]) {
        const uint32_t kb = ks_begin + s * SUBK;
        const uint32_t nrows = (min(ks_end, kb + SUBK) - kb) * 32u;
        if (NORM) {
#pragma unroll
            for (int q = 0; q < XQ; ++q) {
                h8_t ha = __builtin_bit_cast(h8_t, xv[q]);
                const float gq = __half2float(
                    __ushort_as_half((unsigned short)(xb[q][xprod == 5u ? 2 : 0] & 0xffffu)));
#pragma unroll
                for (int e2 = 0; e2 < 8; ++e2) {
                    // element copied to a scalar first: a bit cast of the vector element itself
                    // compiled to a read of element 0 for every e2
                    const _Float16 xe = ha[e2];
                    const __half r = norm_scale(__builtin_bit_cast(__half, xe), xinv[e2], gq);
                    ha[e2] = __builtin_bit_cast(_Float16, r);
                }
                if (xprod == 5u) {
                    // decode token shift of the normalised values (k44_rmsnorm_kernel's
                    // expression and order), and the shifted state for an owned pass
                    const uint32_t rf = a.rf;
                    float mw[4];
                    mw[0] = __half2float(__ushort_as_half((unsigned short)(xb[q][0] & 0xffffu)));
                    mw[1] = __half2float(__ushort_as_half((unsigned short)(xb[q][0] >> 16)));
                    mw[2] = __half2float(__ushort_as_half((unsigned short)(xb[q][1] & 0xffffu)));
                    mw[3] = __half2float(__ushort_as_half((unsigned short)(xb[q][1] >> 16)));
                    const h8_t s0 = __builtin_bit_cast(h8_t, xc[q]);
                    const h8_t s1 = __builtin_bit_cast(h8_t, xs1[q]);
                    const h8_t s2 = __builtin_bit_cast(h8_t, xs2[q]);
                    h8_t y2, n0 = s0, n1 = s1, n2 = s2;
#pragma unroll
                    for (int e2 = 0; e2 < 8; ++e2) {
                        const uint32_t t = (uint32_t)(lane & 1) * 8u + (uint32_t)e2;
                        const _Float16 ne = ha[e2], e0 = s0[e2], e1 = s1[e2], e3 = s2[e2];
                        float acc = mw[0] * (float)ne;
                        acc = fmaf(mw[1], (float)e0, acc);
                        if (rf > 2u) acc = fmaf(mw[2], (float)e1, acc);
                        if (rf > 3u) acc = fmaf(mw[3], (float)e3, acc);
                        const _Float16 yv = __builtin_bit_cast(_Float16, f16_of(acc));
                        const bool live = t < a.sh_tokens;
                        y2[e2] = live ? yv : (_Float16)0.0f;
                        n0[e2] = live ? ne : e0;
                        n1[e2] = live ? e0 : e1;
                        n2[e2] = live ? e1 : e3;
                    }
                    const uint32_t rb = (uint32_t)(32 * (wave + 4 * q));
                    if (rb < nrows && ((ownb >> (s * 16u + (uint32_t)(wave + 4 * q))) & 1u)) {
                        typedef __attribute__((address_space(1))) u4_t gu4w;
                        gu4w *sn = (gu4w *)(a.state_next + (uint64_t)xb[q][3] * (rf - 1u) * 16u +
                                            (uint32_t)(lane & 1) * 8u);
                        sn[0] = __builtin_bit_cast(u4_t, n0);
                        if (rf > 2u) sn[2] = __builtin_bit_cast(u4_t, n1);
                        if (rf > 3u) sn[4] = __builtin_bit_cast(u4_t, n2);
                    }
                    ha = y2;
                }
                xv[q] = __builtin_bit_cast(u4_t, ha);
            }
        } else if (xprod != 0u) {
            // (as fp16 vectors: element access through pointer casts of the u4 registers would
            // put them on the stack)
#pragma unroll
            for (int q = 0; q < XQ; ++q) {
                h8_t ha = __builtin_bit_cast(h8_t, xv[q]);
                const h8_t hb = __builtin_bit_cast(h8_t, xb[q]);
                const h8_t hc = __builtin_bit_cast(h8_t, xc[q]);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float bc = xprod == 3u ? (float)(_Float16)((float)hb[e] * (float)hc[e])
                                                 : (float)hb[e];
                    ha[e] = (_Float16)((float)ha[e] * bc);
                }
                xv[q] = __builtin_bit_cast(u4_t, ha);
            }
        }
#pragma unroll
        for (int q = 0; q < XQ; ++q) {
            const uint32_t rb = (uint32_t)(32 * (wave + 4 * q));
            if (rb < nrows)
                *reinterpret_cast<u4_t *>(&xl[buf][rb + (uint32_t)(lane >> 1)][(lane & 1) * 8]) =
                    xv[q];
        }
    };

    // a folded norm's producer slots first: they arrive ahead of the weights and the gather
    // (loads complete in issue order), so the scales are formed while those are in flight
    // (after the weights where those were issued from the preloaded arguments)
    SlotLoads<16u> slp;
    if constexpr (NORM)
        rms_slots_issue<16u>(reinterpret_cast<const uint64_t *>(a.xslots), a.xslots_n, 0u, slp);
    if (geo == 0u) {
#pragma unroll
        for (int u = 0; u < AF; ++u) load_a((uint32_t)u, af[u]);
    }
    u4_t xv[XQ], xb[XQ], xc[XQ];
    gather(0u, xv, xb, xc);
    // Lane holds C[4g + i][lane & 15]: neuron 16*blk + 4g + i, token lane & 15.  A workgroup
    // that may run the epilogue (whole contraction here, or split-K reduced by the tile's last
    // workgroup) issues its epilogue loads now: cout_map and biases with the first gather, the
    // residuals they address after it (all read-only or written only by this lane's store).
    const int g = lane >> 4;
    const uint32_t t = (uint32_t)(lane & 15);
    const bool epi = !a.part || a.arrive;
    uint32_t j0[BPW];
#pragma unroll
    for (int bi = 0; bi < BPW; ++bi)
        j0[bi] = tile * (uint32_t)NT + 16u * (uint32_t)(wave + 4 * bi) + 4u * (uint32_t)g;
    NarrowEpi<BPW> e;
    uint32_t cb[BPW][4];
    if (epi) narrow_epi_maps<BPW>(a, j0, cb, e);
    // A copy carried for an earlier launch (cp_rows): the thread's first 16 bytes loaded now,
    // stored after the contraction.
    const uint32_t cpn = a.cp_rows * 2u, cpstep = tiles * kgroups * 256u;
    const uint32_t cpe = local * 256u + (uint32_t)tid;
    auto cp_at = [&](const __half *base, uint32_t stride, uint32_t i) {
        return base + (uint64_t)(i >> 1) * stride + (i & 1u) * 8u;
    };
    u4_t cpv = {0u, 0u, 0u, 0u};
    if (cpn) cpv = *(gu4_t *)cp_at(a.cp_src, a.cp_sstride, min(cpe, cpn - 1u));
    if constexpr (NORM) {
        __shared__ uint4 ipart[4][16];
        __shared__ float sinv[16];
        rms_slots_finish<16u>(slp, reinterpret_cast<const uint64_t *>(a.xslots), a.xslots_n, 0u,
                              a.norm_D, a.norm_eps, ipart, sinv);
#pragma unroll
        for (int e2 = 0; e2 < 8; ++e2) xinv[e2] = sinv[(lane & 1) * 8 + e2];
    }
    store(0u, 0, xv, xb, xc);
    if (epi) narrow_epi_res<BPW>(a, j0, t, cb, e);
    __syncthreads();

    const int tr_row = 8 * g + ((lane & 15) >> 2);
    const int tr_col = 4 * (lane & 3);
    f4_t acc[BPW];
#pragma unroll
    for (int i = 0; i < BPW; ++i) acc[i] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

    for (uint32_t s = 0; s < nsub; ++s) {
        const int buf = (int)(s & 1u);
        const bool more = s + 1u < nsub;
        if (more) gather(s + 1u, xv, xb, xc);
        const uint32_t kb = ks_begin + s * SUBK;
#pragma unroll
        for (int u = 0; u < SUBK; ++u) {
            const uint32_t k2 = kb + (uint32_t)u;
            if (k2 < ks_end) {
                const _Float16 *p = &xl[buf][u * 32 + tr_row][tr_col];
                const h4_t lo = lds_read_tr16(p);
                const h4_t hi = lds_read_tr16(p + 4 * NARROW_PITCH);
                const h8_t b = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
                for (int i = 0; i < BPW; ++i)
                    acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[u][i], b, acc[i], 0, 0, 0);
            }
            load_a(k2 - ks_begin + (uint32_t)AF, af[u]);  // next sub-chunk's fragment (or none)
        }
        if (more) {
            store(s + 1u, buf ^ 1, xv, xb, xc);
            __syncthreads();
        }
    }

    if (cpn) {
        typedef __attribute__((address_space(1))) u4_t gu4w;
        auto dst = [&](uint32_t i) { return (gu4w *)cp_at(a.cp_dst, a.cp_dstride, i); };
        if (cpe < cpn) *dst(cpe) = cpv;
        for (uint32_t i = cpe + cpstep; i < cpn; i += cpstep)
            *dst(i) = *(gu4_t *)cp_at(a.cp_src, a.cp_sstride, i);
    }
    if (epi) {
        // the fused epilogue (loads issued above), then the tile's share of a folded RMSNorm
        uint16_t out[BPW][4];
        if (a.part && !narrow_reduce_last<BPW>(a, acc, j0, t, tile, zgroup)) return;
        narrow_epi_store<BPW>(a, acc, e, out);
        if (a.norm_part) narrow_norm_publish<BPW>(a, e, out, tile);
        return;
    }
#pragma unroll
    for (int bi = 0; bi < BPW; ++bi) {
        const uint32_t blk = (uint32_t)(wave + 4 * bi);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t j = tile * (uint32_t)NT + 16u * blk + 4u * (uint32_t)g + (uint32_t)i;
            a.part[((uint64_t)zgroup * a.cout + j) * 16u + t] = acc[bi][i];
        }
    }
}

// Set-up probe of the XCD-local split-K meeting: workgroup b records the XCD it runs on.
__global__ __launch_bounds__(64) void k44_xcd_probe_kernel(uint32_t *out) {
    if (threadIdx.x == 0u) out[blockIdx.x] = k44_xcc_id();
}

hipError_t launch_xcd_probe(uint32_t *out, uint32_t n, hipStream_t stream) {
    if (n == 0u) return hipSuccess;
    hipLaunchKernelGGL(k44_xcd_probe_kernel, dim3(n), dim3(64), 0, stream, out);
    return hipGetLastError();
}

hipError_t launch_mfma_narrow(const MfmaGroup &g, uint32_t nt, uint32_t items,
                              hipStream_t stream, uint32_t prod, uint32_t max_items,
                              const NarrowPre &pre) {
    if (prod != 0u && ((nt != 64u && nt != 128u) || (prod < 2u || prod > 5u)))
        return hipErrorInvalidValue;
    if (items == 0u) return hipSuccess;
    const dim3 grid(items), block(256);
    // 64/128-neuron tiles: grid (max_items, waves) when it launches at most 1.5x the
    // workgroups (max_items = the largest wave's workgroups; 0 = not known).
    const bool byy = max_items != 0u && 2ull * max_items * g.n <= 3ull * items;
    const dim3 grid_y(max_items, g.n);
    // a wave past the group's count never selects its preloaded entry
    NarrowPre p = pre;
    for (uint32_t i = g.n; i < (uint32_t)NarrowPre::N; ++i) p.geo[i] = 0u;
    if (g.n > 255u || p.shift > 40u) return hipErrorInvalidValue;
    const uint32_t nsh = g.n | (p.shift << 8);
#define K44_PRE_ARGS                                                                         \
    g.waves, g.start, nsh, p.geo[0], p.geo[1], p.geo[2], p.geo[3], p.geo[4], p.geo[5], p.base
#define K44_NL(N, P)                                                                               \
    if (byy)                                                                                       \
        hipLaunchKernelGGL((k44_mfma_narrow_long_kernel<N, P, true>), grid_y, block, 0, stream, \
                           K44_PRE_ARGS);                                                          \
    else                                                                                           \
        hipLaunchKernelGGL((k44_mfma_narrow_long_kernel<N, P, false>), grid, block, 0, stream,     \
                           K44_PRE_ARGS);
    switch (nt) {
    case 16u: hipLaunchKernelGGL(k44_mfma_narrow_kernel<16>, grid, block, 0, stream, K44_GROUP_ARGS(g)); break;
    case 32u: hipLaunchKernelGGL(k44_mfma_narrow_kernel<32>, grid, block, 0, stream, K44_GROUP_ARGS(g)); break;
    case 64u:
        if (prod == 5u) {
            K44_NL(64, 5)
        } else if (prod == 4u) {
            K44_NL(64, 4)
        } else if (prod == 3u) {
            K44_NL(64, 3)
        } else if (prod == 2u) {
            K44_NL(64, 2)
        } else {
            K44_NL(64, 0)
        }
        break;
    case 128u:
        if (prod == 5u) {
            K44_NL(128, 5)
        } else if (prod == 4u) {
            K44_NL(128, 4)
        } else if (prod == 3u) {
            K44_NL(128, 3)
        } else if (prod == 2u) {
            K44_NL(128, 2)
        } else {
            K44_NL(128, 0)
        }
        break;
    default: return hipErrorInvalidValue;
    }
#undef K44_NL
#undef K44_PRE_ARGS
    return hipGetLastError();
}

}  // namespace k44dev
