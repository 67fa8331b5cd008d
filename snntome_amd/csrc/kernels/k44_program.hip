// Translation unit of the decode program kernel (k44_program.hpp describes the execution model).
#include "k44_program.hpp"

#include <type_traits>

#include "k44_mfma_tile.hpp"
#include "k44_sumsq.hpp"

namespace k44dev {

namespace {

typedef __attribute__((address_space(1))) unsigned long long gu64;
typedef __attribute__((address_space(1))) uint32_t gu32;

// Device-coherent 8-byte accesses (agent-scope relaxed atomics: the loads miss stale lines of
// this XCD's caches, the stores are not left dirty in them).
__device__ __forceinline__ uint64_t cld8(const void *p) {
    return __hip_atomic_load((const gu64 *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void cst8(void *p, uint64_t v) {
    __hip_atomic_store((gu64 *)p, (unsigned long long)v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Cached loads (data read-only in the launch, or written once per launch before it is read).
__device__ __forceinline__ uint64_t ld8(const void *p) {
    return *(const __attribute__((address_space(1))) uint64_t *)p;
}
__device__ __forceinline__ u4_t ld16(const void *p) {
    return *(const __attribute__((address_space(1))) u4_t *)p;
}
__device__ __forceinline__ void cst16(void *p, u4_t v) {
    cst8(p, (uint64_t)v[0] | ((uint64_t)v[1] << 32));
    cst8((char *)p + 8, (uint64_t)v[2] | ((uint64_t)v[3] << 32));
}

constexpr uint32_t PW_ROWS = 256;   // rows of one 8-k-step chunk (per wave)
constexpr uint32_t PW_PITCH = 24;   // halves per LDS row: 16 tokens + 8 skew

struct ProgLds {
    union {
        _Float16 xl[4][PW_ROWS][PW_PITCH];  // PROG_WAVES: each wave's X rows of one chunk
        uint4 npart[4][2][8];               // PROG_NORM: per-wave token sums (limbs, flags)
        _Float16 et[16][136];               // PROG_EMBED: [token][channel] block
        uint64_t kpart[4][2][8];            // PROG_ARGMAX: per-wave token keys
    } u;
    f4_t red[2][4][64];  // PROG_WAVES: the 4 waves' accumulators of each block
    uint4 ipart[4][16];  // per-wave token sums of the norm slots
    float inv[16];    // per-token RMSNorm scales
    uint32_t inv_stage;  // 1 + the stage whose scales inv holds (0: none)
    uint32_t flag;
    uint32_t last;
    uint64_t t_wait;  // trace: when the last wait of this workgroup was released
    uint64_t t_mark[3];  // trace (projection items): inputs arrived, MFMAs done, stores done
};

// Waits (whole workgroup) until stage s - 1 has signalled every item.  Returns false when the
// program is aborted (a wait past the time limit, here or in another workgroup).
__device__ __forceinline__ bool prog_wait(const ProgArgs &p, uint32_t s, uint32_t &known, ProgLds &L) {
    if (s == 0u || known >= s) {
        if (p.trace && threadIdx.x == 0u) L.t_wait = wall_clock64();
        return true;
    }
    if (threadIdx.x == 0u) {
        const uint32_t target = p.stages[s - 1u].items;
        uint32_t ok = 1u;
        const uint64_t t0 = wall_clock64();
        for (;;) {
            if (__hip_atomic_load((const gu32 *)(p.done + s - 1u), __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT) >= target)
                break;
            if (__hip_atomic_load((const gu32 *)p.abort, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT) != 0u) {
                ok = 0u;
                break;
            }
            if (wall_clock64() - t0 > p.spin_ticks) {
                __hip_atomic_store((gu32 *)p.abort, s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ok = 0u;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        L.flag = ok;
        if (p.trace) L.t_wait = wall_clock64();
    }
    __syncthreads();
    const bool ok = L.flag != 0u;
    __syncthreads();  // the flag is written again by a later wait
    if (ok) known = s;
    return ok;
}

// Item done: every wave's stores performed, then one count at stage s.
__device__ __forceinline__ void prog_signal(const ProgArgs &p, uint32_t s, ProgLds &L) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (p.trace && threadIdx.x == 0u) L.t_mark[2] = wall_clock64();
    __syncthreads();
    if (threadIdx.x == 0u)
        __hip_atomic_fetch_add((gu32 *)(p.done + s), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Per-token RMSNorm scales of the norm whose producers stored n item slots (16 tokens x 2 words
// each) into L.inv[0..15]: the whole workgroup adds the slots (exact, so any order gives the
// norm kernel's scales), once per workgroup and stage (L.inv_stage).
__device__ __forceinline__ void prog_inv_from_slots(const uint64_t *slots, uint32_t n, uint32_t D,
                                                    float eps, uint32_t s, ProgLds &L) {
    if (L.inv_stage == s + 1u) return;  // uniform: formed by an earlier item of this stage
    const uint32_t tk = threadIdx.x & 15u, part = threadIdx.x >> 4;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    SumSq q = sumsq_zero();
    for (uint32_t i0 = part; i0 < n; i0 += 64u) {
        uint64_t a[4], b[4];
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
            const uint32_t i = min(i0 + 16u * u, n - 1u);
            a[u] = ld8(slots + ((uint64_t)i * 16u + tk) * 2u);
            b[u] = ld8(slots + ((uint64_t)i * 16u + tk) * 2u + 1u);
        }
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u)
            if (i0 + 16u * u < n) {
                q.l0 += a[u] & 0xffffffffull;
                q.l1 += a[u] >> 32;
                q.l2 += b[u] & 0xffffffffull;
                q.sp |= (uint32_t)(b[u] >> 32);
            }
    }
    q = sumsq_wave_reduce(q, 16);  // the 4 lanes of each token in this wave
    if (lane < 16u) L.ipart[wave][lane] = uint4{(uint32_t)q.l0, (uint32_t)q.l1, (uint32_t)q.l2, q.sp};
    __syncthreads();
    if (threadIdx.x < 16u) {
        SumSq t = sumsq_zero();
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint4 x = L.ipart[v][threadIdx.x];
            t.l0 += x.x;
            t.l1 += x.y;
            t.l2 += x.z;
            t.sp |= x.w;
        }
        L.inv[threadIdx.x] = rms_inv(t, D, eps);
    }
    if (threadIdx.x == 0u) L.inv_stage = s + 1u;
    __syncthreads();
}

// ---------------------------------------------------------------------------------------------
// PROG_WAVES: item = (wave, NT-neuron tile, BPB consecutive 16-neuron blocks), whole
// contraction.  Wave v of the workgroup takes k-steps [v * kq, (v + 1) * kq) (kq =
// ceil(ksteps / 4)) in chunks of 8 (256 rows: its X rows go to its own LDS buffer, read with
// ds_read_b64_tr_b16 as in the narrow kernels) for every block of the item.  Before the wait the
// item requests the A fragments of its first HOLD chunks and the segment starts of its rows
// (read-only); later chunks' fragments replace consumed ones.  Gather forms (uniform per stage)
// as MfmaTileArgs::xprod: 0 plain, 2 fp16(A*B), 3 fp16(A*fp16(B*C)), 4 folded RMSNorm
// fp16(x * inv[t] * gamma[c]).  The 4 waves' fp32 tiles are summed in wave order; wave b runs
// the epilogue of block b (lane = 4 * neuron + token quad: bias, activation, residual or
// cout_map, fp16 RNE, one 8-byte store) and, when a folded RMSNorm reads the output, stores the
// exact sums of squares of what it stored in the item's slot.  PROD, HOLD (A-fragment chunks
// held in registers) and BPB (blocks per item, 1 or 2) are compile-time: one copy of the code
// per form keeps every row in registers and the code small enough for the instruction cache.
template <uint32_t PROD, uint32_t HOLD, uint32_t BPB>
__device__ __forceinline__ void prog_waves_item(const ProgArgs &p, const ProgStage &st,
                                                uint32_t item, uint32_t s, uint32_t &known,
                                                bool &stop, ProgLds &L) {
    static_assert(HOLD * BPB <= 2u, "A fragments of at most 16 k-steps x 16 neurons per wave");
    uint32_t wi = st.first;
    for (uint32_t k = 1u; k < st.count; ++k)
        if (item >= p.waves[st.first + k].item0) wi = st.first + k;
    const ProgWave w = p.waves[wi];
    const uint32_t local = item - w.item0;
    const uint32_t ipt = w.nb / BPB;  // items per tile
    const uint32_t tile = local / ipt, blk0 = (local - tile * ipt) * BPB;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t kq = (w.ksteps + 3u) >> 2;
    const uint32_t k0 = min(w.ksteps, wave * kq), k1 = min(w.ksteps, k0 + kq);
    const uint32_t klast = k1 > k0 ? k1 - 1u : 0u;
    const uint32_t nchunks = (k1 - k0 + 7u) >> 3;

    typedef const __attribute__((address_space(1))) h8_t gh8;
    gh8 *wf = (gh8 *)(reinterpret_cast<const h8_t *>(w.Wf) +
                      ((uint64_t)tile * w.ksteps * w.nb + blk0) * 64u + lane);
    const uint64_t kstride = (uint64_t)w.nb * 64u;
    h8_t af[HOLD][8][BPB];
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
        for (uint32_t b = 0; b < BPB; ++b)
            af[0][u][b] = __builtin_nontemporal_load(
                wf + (uint64_t)min(k0 + (uint32_t)u, klast) * kstride + 64u * b);
    if constexpr (HOLD > 1u)
        if (nchunks > 1u)
#pragma unroll
            for (int u = 0; u < 8; ++u)
                af[HOLD - 1u][u][0] = __builtin_nontemporal_load(
                    wf + (uint64_t)min(k0 + 8u + (uint32_t)u, klast) * kstride);

    // Epilogue operands of wave eb < BPB (lane = 4 * n + q: neuron n of block blk0 + eb,
    // tokens 4q..4q+3).
    const uint32_t en = lane >> 2, eq = lane & 3u;
    const bool epi = wave < BPB;
    const uint32_t j = tile * 16u * w.nb + (blk0 + (epi ? wave : 0u)) * 16u + en;
    uint64_t o = j;
    uint32_t bbits = 0u;
    bool empty = false;
    if (epi) {
        if (w.cmap) {
            const uint32_t m = w.cmap[j];
            empty = m == 0xffffu;
            o = m;
        }
        if (w.bias) bbits = reinterpret_cast<const uint16_t *>(w.bias)[j];
    }
    // Canvas offsets of this lane's rows in the first chunk (segment starts are read-only).
    const kconst_u64 *segr = (const kconst_u64 *)(w.seg) + (uint64_t)tile * w.K;
    auto row_off = [&](uint32_t k) -> uint64_t {  // row 32k + lane/2, token half lane & 1
        const uint32_t r = k * 32u;
        const uint32_t sg = r / w.S;
        return segr[sg] + (uint64_t)(r - sg * w.S) * w.step + (uint64_t)(lane >> 1) * w.step +
               (uint64_t)(lane & 1u) * 8u;
    };
    uint64_t off0[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) off0[u] = row_off(min(k0 + (uint32_t)u, klast));
    typedef const __attribute__((address_space(1))) uint16_t gu16;
    auto gamma_of = [&](uint64_t off) -> uint32_t {
        const uint64_t row = off - (uint64_t)(lane & 1u) * 8u;
        return w.xgamma ? (uint32_t)((gu16 *)w.xgamma)[(row - w.xg_base) >> w.xg_shift] : 0x3c00u;
    };
    uint32_t gb[PROD == 4u ? 8 : 1];
    if constexpr (PROD == 4u)
#pragma unroll
        for (int u = 0; u < 8; ++u) gb[u] = gamma_of(off0[u]);

    if (!prog_wait(p, s, known, L)) {
        stop = true;
        return;
    }

    // Inputs written by earlier stages: residual, X rows, then the norm scales.
    uint64_t rbits = 0u;
    const uint64_t yo = o * w.out_stride + 4u * eq;
    if (epi && w.R && !empty) rbits = ld8(w.R + yo);
    u4_t va[8], vb[PROD == 2u || PROD == 3u ? 8 : 1], vc[PROD == 3u ? 8 : 1];
    // X rows of chunk c (offsets: the first chunk's were formed before the wait).  One
    // straight-line loop per gather form (a form test per row would make the compiler keep the
    // rows in memory and wait for each load).
    auto gather = [&](uint32_t c) {
        uint64_t off[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            off[u] = c == 0u ? off0[u] : row_off(min(k0 + 8u * c + (uint32_t)u, klast));
        if constexpr (PROD == 4u) {
            if (c != 0u)
#pragma unroll
                for (int u = 0; u < 8; ++u) gb[u] = gamma_of(off[u]);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            va[u] = ld16(w.Xo[0] + off[u]);
            if constexpr (PROD == 2u || PROD == 3u) vb[u] = ld16(w.Xo[1] + off[u]);
            if constexpr (PROD == 3u) vc[u] = ld16(w.Xo[2] + off[u]);
        }
    };
    if (nchunks) gather(0u);
    if constexpr (PROD == 4u) prog_inv_from_slots(w.slot_in, w.slot_n, w.norm_D, w.norm_eps, s, L);
    float xinv[PROD == 4u ? 8 : 1];
    if constexpr (PROD == 4u)
#pragma unroll
        for (int e = 0; e < 8; ++e) xinv[e] = L.inv[(lane & 1u) * 8u + (uint32_t)e];

    _Float16(*xl)[PW_PITCH] = L.u.xl[wave];
    auto store = [&]() {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            h8_t ha = __builtin_bit_cast(h8_t, va[u]);
            if constexpr (PROD == 4u) {
                const float gq = __half2float(__ushort_as_half((unsigned short)gb[u]));
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const _Float16 xe = ha[e];
                    const __half r = norm_scale(__builtin_bit_cast(__half, xe), xinv[e], gq);
                    ha[e] = __builtin_bit_cast(_Float16, r);
                }
            } else if constexpr (PROD == 2u) {
                const h8_t hb = __builtin_bit_cast(h8_t, vb[u]);
#pragma unroll
                for (int e = 0; e < 8; ++e) ha[e] = (_Float16)((float)ha[e] * (float)hb[e]);
            } else if constexpr (PROD == 3u) {
                const h8_t hb = __builtin_bit_cast(h8_t, vb[u]);
                const h8_t hc = __builtin_bit_cast(h8_t, vc[u]);
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    ha[e] = (_Float16)((float)ha[e] * (float)(_Float16)((float)hb[e] * (float)hc[e]));
            }
            *reinterpret_cast<u4_t *>(&xl[32 * u + (int)(lane >> 1)][(lane & 1u) * 8u]) =
                __builtin_bit_cast(u4_t, ha);
        }
        // the wave's own transposed reads below see these rows
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    };

    const int g = (int)(lane >> 4);
    const int tr_row = 8 * g + (int)((lane & 15u) >> 2);
    const int tr_col = 4 * (int)(lane & 3u);
    f4_t acc[BPB];
#pragma unroll
    for (uint32_t b = 0; b < BPB; ++b) acc[b] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // (the register set is a compile-time index: a runtime one would put af on the stack)
    auto mfma_chunk = [&](uint32_t c, auto set) {
        h8_t(&f)[8][BPB] = af[decltype(set)::value];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const uint32_t k = k0 + 8u * c + (uint32_t)u;
            if (k < k1) {
                const _Float16 *pp = &xl[32 * u + tr_row][tr_col];
                const h4_t lo = lds_read_tr16(pp);
                const h4_t hi = lds_read_tr16(pp + 4 * PW_PITCH);
                const h8_t bx = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
                for (uint32_t b = 0; b < BPB; ++b)
                    acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f[u][b], bx, acc[b], 0, 0, 0);
            }
            // fragment HOLD chunks ahead (contractions longer than the registers hold)
            if (c + HOLD < nchunks)
#pragma unroll
                for (uint32_t b = 0; b < BPB; ++b)
                    f[u][b] = __builtin_nontemporal_load(
                        wf + (uint64_t)min(k + 8u * HOLD, klast) * kstride + 64u * b);
        }
    };
    for (uint32_t c = 0; c < nchunks; ++c) {
        store();
        if (p.trace && threadIdx.x == 0u && c == 0u) L.t_mark[0] = wall_clock64();
        if (c + 1u < nchunks) gather(c + 1u);  // in flight during the MFMAs
        if (HOLD > 1u && (c & 1u))
            mfma_chunk(c, std::integral_constant<int, HOLD - 1>{});
        else
            mfma_chunk(c, std::integral_constant<int, 0>{});
        // the next chunk's rows overwrite this one's only after its reads
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }

#pragma unroll
    for (uint32_t b = 0; b < BPB; ++b) L.red[b][wave][lane] = acc[b];
    __syncthreads();
    if (p.trace && threadIdx.x == 0u) L.t_mark[1] = wall_clock64();
    if (epi) {
        // element (n, t) of block `wave` sits in lane 16 * (n / 4) + t, component n % 4
        float v[4];
        const uint32_t comp = en & 3u;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t src = (en >> 2) * 16u + 4u * eq + (uint32_t)e;
            float a = L.red[wave][0][src][comp];
            a += L.red[wave][1][src][comp];
            a += L.red[wave][2][src][comp];
            a += L.red[wave][3][src][comp];
            v[e] = a;
        }
        const float b = w.bias ? __half2float(__ushort_as_half((unsigned short)bbits)) : 0.0f;
        uint16_t out[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float r = w.R ? __half2float(__ushort_as_half((unsigned short)(rbits >> (16 * e))))
                                : 0.0f;
            const float x = v[e] + b;
            out[e] = __half_as_ushort(
                __float2half_rn(w.cmap ? apply_act(x + r, w.act) : apply_act(x, w.act) + r));
        }
        if (!empty) {
            const uint64_t ov = (uint64_t)out[0] | ((uint64_t)out[1] << 16) |
                                ((uint64_t)out[2] << 32) | ((uint64_t)out[3] << 48);
            cst8(w.Ys + yo, ov);
            cst8(w.Y + yo, ov);
        }
        if (w.slot_out) {
            // tokens 4q + e: sums over the 16 neurons of the block (lanes sharing q), exact;
            // lane q of neuron 0 stores tokens 4q..4q+3 of the block's slot
            uint64_t *slot = w.slot_out + ((uint64_t)item * BPB + wave) * 32u;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                SumSq q = sumsq_zero();
                if (!empty) sumsq_add(q, out[e]);
                q = sumsq_wave_reduce(q, 4);
                if (en == 0u) {
                    const uint32_t t = 4u * eq + (uint32_t)e;
                    cst8(slot + 2u * t, q.l0 | (q.l1 << 32));
                    cst8(slot + 2u * t + 1u, q.l2 | ((uint64_t)q.sp << 32));
                }
            }
        }
    }
    prog_signal(p, s, L);
}

// ---------------------------------------------------------------------------------------------
// PROG_NORM: item = 128 channels x the first 16 token columns; thread = (channel, token octet).
// y = fp16(x * inv[t] * gamma[c]) with the RMSNorm kernel's expression; inv from the producers'
// slots or summed here over all D channels (exact, so the same bits either way).  With a decode
// token shift (y2, rf 1..5): y2 = mu[c][0] * y + sum_i mu[c][i] * state[c][i-1][t] and the state
// shifted, with the arithmetic of k44_rmsnorm_kernel<1, RF>; octets at or past `tokens` get
// y2 = 0 (the whole stride, as that kernel writes) and no y or state.
constexpr uint32_t PN_RF = 5u;  // largest receptive field of the program's token shift
__device__ __forceinline__ void prog_norm_item(const ProgArgs &p, const ProgAux &a, uint32_t item,
                                               uint32_t s, uint32_t &known, bool &stop,
                                               ProgLds &L) {
    const uint32_t cl = threadIdx.x >> 1, h = threadIdx.x & 1u;
    const uint32_t c = item * 128u + cl;
    const bool live = c < a.D;
    const uint32_t cc = live ? c : a.D - 1u;
    const uint32_t t0 = h * 8u;
    const bool octet_live = t0 < a.tokens;
    const uint32_t rf = a.y2 ? a.rf : 0u;
    const uint32_t gbits = a.table ? (uint32_t)reinterpret_cast<const uint16_t *>(a.table)[cc] : 0x3c00u;
    // mixing weights and the channel's state rows (read-only here): requested before the wait
    uint32_t mbits[PN_RF];
    uint4 sv[PN_RF - 1u];
    {
        const uint16_t *m = reinterpret_cast<const uint16_t *>(a.mu) + (uint64_t)cc * rf;
        const __half *st = a.state + (uint64_t)cc * (rf - 1u) * 64u + t0;
#pragma unroll
        for (uint32_t i = 0; i < PN_RF; ++i) {
            mbits[i] = i < rf ? (uint32_t)m[i] : 0u;
            if (i >= 1u) sv[i - 1] = i < rf ? *reinterpret_cast<const uint4 *>(st + (i - 1u) * 64u)
                                            : uint4{0u, 0u, 0u, 0u};
        }
    }
    if (!prog_wait(p, s, known, L)) {
        stop = true;
        return;
    }
    const u4_t xo = ld16(a.x + (uint64_t)cc * a.stride + t0);
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    if (a.slot_in) {
        prog_inv_from_slots(a.slot_in, a.slot_n, a.D, a.eps, s, L);
    } else {
        SumSq ss[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) ss[e] = sumsq_zero();
        for (uint32_t ch = cl; ch < a.D; ch += 2u * 128u) {
            const u4_t v0 = ld16(a.x + (uint64_t)ch * a.stride + t0);
            const u4_t v1 = ld16(a.x + (uint64_t)min(ch + 128u, a.D - 1u) * a.stride + t0);
            const bool two = ch + 128u < a.D;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                sumsq_add(ss[e], v0[e >> 1] >> (16 * (e & 1)));
                sumsq_add(ss[e], two ? v1[e >> 1] >> (16 * (e & 1)) : 0u);
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const SumSq q = sumsq_wave_reduce(ss[e], 2);  // lanes sharing the octet
            if (lane < 2u)
                L.u.npart[wave][lane][e] = uint4{(uint32_t)q.l0, (uint32_t)q.l1, (uint32_t)q.l2, q.sp};
        }
        __syncthreads();
        if (threadIdx.x < 16u) {
            const uint32_t hh = threadIdx.x >> 3, e = threadIdx.x & 7u;
            SumSq q = sumsq_zero();
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint4 x = L.u.npart[v][hh][e];
                q.l0 += x.x;
                q.l1 += x.y;
                q.l2 += x.z;
                q.sp |= x.w;
            }
            L.inv[threadIdx.x] = rms_inv(q, a.D, a.eps);
        }
        __syncthreads();
    }
    if (live) {
        const h8_t xh = __builtin_bit_cast(h8_t, xo);
        const float go = __half2float(__ushort_as_half((unsigned short)gbits));
        h8_t oh;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            // element copied to a scalar first (a bit cast of the vector element itself has
            // compiled to a read of element 0 for every e)
            const _Float16 xe = xh[e];
            oh[e] = __builtin_bit_cast(_Float16, norm_scale(__builtin_bit_cast(__half, xe),
                                                            L.inv[t0 + (uint32_t)e], go));
        }
        // y of octets that hold requests only (the stand-alone kernel's grid)
        if (octet_live) {
            cst16(a.ys + (uint64_t)c * a.stride + t0, __builtin_bit_cast(u4_t, oh));
            cst16(a.y + (uint64_t)c * a.stride + t0, __builtin_bit_cast(u4_t, oh));
        }
        if (rf) {
            h8_t y2 = {};
            if (octet_live) {
                uint4 nsv[PN_RF - 1u];
#pragma unroll
                for (uint32_t i = 1; i < PN_RF; ++i) nsv[i - 1] = sv[i - 1];
                float mw[PN_RF];
#pragma unroll
                for (uint32_t i = 0; i < PN_RF; ++i)
                    mw[i] = __half2float(__ushort_as_half((unsigned short)mbits[i]));
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    if (t0 + (uint32_t)e >= a.tokens) {
                        y2[e] = (_Float16)0.0f;
                        continue;
                    }
                    float acc = mw[0] * (float)oh[e];
#pragma unroll
                    for (uint32_t i = 1; i < PN_RF; ++i)
                        if (i < rf)
                            acc = fmaf(mw[i], __half2float(reinterpret_cast<const __half *>(&sv[i - 1])[e]), acc);
                    y2[e] = __builtin_bit_cast(_Float16, f16_of(acc));
#pragma unroll
                    for (uint32_t i = PN_RF - 1u; i > 1u; --i)
                        if (i < rf)
                            reinterpret_cast<__half *>(&nsv[i - 1])[e] =
                                reinterpret_cast<const __half *>(&sv[i - 2])[e];
                    if (rf > 1u) reinterpret_cast<_Float16 *>(&nsv[0])[e] = oh[e];
                }
                __half *stw = a.state + (uint64_t)c * (rf - 1u) * 64u + t0;
#pragma unroll
                for (uint32_t i = 1; i < PN_RF; ++i)
                    if (i < rf) cst16(stw + (i - 1u) * 64u, __builtin_bit_cast(u4_t, nsv[i - 1]));
            }
            __half *y2r = a.y2 + (uint64_t)c * a.stride;
            cst16(a.y2s + (uint64_t)c * a.stride + t0, __builtin_bit_cast(u4_t, y2));
            cst16(y2r + t0, __builtin_bit_cast(u4_t, y2));
            // octets 2..stride/8-1 (no requests): zeros, as the stand-alone kernel writes them
            for (uint32_t oc = 2u + h; oc < a.stride / 8u; oc += 2u)
                cst16(y2r + 8u * oc, u4_t{0u, 0u, 0u, 0u});
        }
    }
    prog_signal(p, s, L);
}

// ---------------------------------------------------------------------------------------------
// PROG_EMBED: item = 128 channels; y[c][t] = table[id[t]][c] for t < tokens (ids below vocab),
// 0 elsewhere in the stride (as k44_embed_vec_kernel writes).
__device__ __forceinline__ void prog_embed_item(const ProgArgs &p, const ProgAux &a, uint32_t item, uint32_t s,
                                uint32_t &known, bool &stop, ProgLds &L) {
    const uint32_t tt = threadIdx.x >> 4, cg = threadIdx.x & 15u;
    const uint32_t c0 = item * 128u, c = c0 + 8u * cg;
    const uint32_t id = a.ids_in[tt < a.tokens ? tt : 0u];
    const bool ok = tt < a.tokens && id < a.vocab && c < a.D;
    const uint64_t row = id < a.vocab ? id : 0u;
    const uint4 v = *reinterpret_cast<const uint4 *>(a.table + row * a.D + (c < a.D ? c : 0u));
    if (!prog_wait(p, s, known, L)) {
        stop = true;
        return;
    }
    *reinterpret_cast<uint4 *>(&L.u.et[tt][8u * cg]) = ok ? v : uint4{0u, 0u, 0u, 0u};
    __syncthreads();
    const uint32_t cl = threadIdx.x >> 1, h = threadIdx.x & 1u;
    if (c0 + cl < a.D) {
        h8_t o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = L.u.et[8u * h + (uint32_t)e][cl];
        __half *yr = a.y + (uint64_t)(c0 + cl) * a.stride;
        cst16(a.ys + (uint64_t)(c0 + cl) * a.stride + 8u * h, __builtin_bit_cast(u4_t, o));
        cst16(yr + 8u * h, __builtin_bit_cast(u4_t, o));
        for (uint32_t oc = 2u + h; oc < a.stride / 8u; oc += 2u) cst16(yr + 8u * oc, u4_t{0u, 0u, 0u, 0u});
    }
    prog_signal(p, s, L);
}

// ---------------------------------------------------------------------------------------------
// PROG_ARGMAX: item = 128 channels of the logits; per token the largest value (lowest channel on
// ties, NaN never chosen, -0 == +0), as k44_argmax_*_kernel: key = (orderable fp16 bits << 32) |
// (0xffffffff - channel), merged by 64-bit atomic maxima (0: no value yet).
__device__ __forceinline__ uint64_t amax_key(uint32_t hb, uint32_t ch) {
    hb &= 0xffffu;
    if ((hb & 0x7fffu) > 0x7c00u) return 0ull;  // NaN
    if (hb == 0x8000u) hb = 0u;                  // -0 ties with +0
    const uint32_t ord = (hb & 0x8000u) ? (~hb & 0xffffu) : (hb | 0x8000u);
    return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - ch);
}

__device__ __forceinline__ uint64_t shfl_max_u64(uint64_t v, int m) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, m, 64);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), m, 64);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    return o > v ? o : v;
}

__device__ __forceinline__ void prog_argmax_item(const ProgArgs &p, const ProgAux &a, uint32_t item, uint32_t s,
                                 uint32_t &known, bool &stop, ProgLds &L) {
    const uint32_t rl = threadIdx.x >> 1, h = threadIdx.x & 1u;
    const uint32_t r = item * 128u + rl;
    if (!prog_wait(p, s, known, L)) {
        stop = true;
        return;
    }
    uint64_t key[8];
    u4_t v = {0u, 0u, 0u, 0u};
    if (r < a.D) v = ld16(a.x + (uint64_t)r * a.stride + 8u * h);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t t = 8u * h + (uint32_t)e;
        key[e] = (r < a.D && t < a.tokens) ? amax_key(v[e >> 1] >> (16 * (e & 1)), r) : 0ull;
#pragma unroll
        for (int m = 2; m < 64; m <<= 1) key[e] = shfl_max_u64(key[e], m);
    }
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    if (lane < 2u)
#pragma unroll
        for (int e = 0; e < 8; ++e) L.u.kpart[wave][lane][e] = key[e];
    __syncthreads();
    if (threadIdx.x < 16u) {
        const uint32_t hh = threadIdx.x >> 3, e = threadIdx.x & 7u;
        uint64_t k = L.u.kpart[0][hh][e];
#pragma unroll
        for (int q = 1; q < 4; ++q) k = L.u.kpart[q][hh][e] > k ? L.u.kpart[q][hh][e] : k;
        if (k)
            __hip_atomic_fetch_max((gu64 *)(a.keys + threadIdx.x), (unsigned long long)k,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    prog_signal(p, s, L);
}

// PROG_ARGMAX_FINAL: ids[t] = channel of key[t] (0 when no value), appended to the history
// while the step counter is below hist_steps; the counter is then incremented.
__device__ __forceinline__ void prog_argmax_final_item(const ProgArgs &p, const ProgAux &a, uint32_t s,
                                       uint32_t &known, bool &stop, ProgLds &L) {
    if (!prog_wait(p, s, known, L)) {
        stop = true;
        return;
    }
    const uint32_t step = a.history ? *a.step_ctr : 0u;
    const uint32_t t = threadIdx.x;
    if (t < a.tokens) {
        const uint64_t k = cld8(a.keys + t);
        const uint32_t id = k ? 0xffffffffu - (uint32_t)k : 0u;
        a.ids_out[t] = id;
        if (a.history && step < a.hist_steps) a.history[(uint64_t)step * a.tokens + t] = id;
    }
    __syncthreads();
    if (a.history && threadIdx.x == 0u) *a.step_ctr = step + 1u;
    prog_signal(p, s, L);
}

// Last workgroup out: every other workgroup has made its last access, so the counters, sums
// and keys return to zero for the next launch.
__device__ __forceinline__ void prog_exit(const ProgArgs &p, ProgLds &L) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0u)
        L.last = __hip_atomic_fetch_add((gu32 *)p.exit_ctr, 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1u;
    __syncthreads();
    if (!L.last) return;
    for (uint32_t i = threadIdx.x; i < p.nstages; i += 256u)
        __hip_atomic_store((gu32 *)(p.done + i), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (uint32_t i = threadIdx.x; i < p.zero_words; i += 256u) cst8(p.zero_base + i, 0ull);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0u)
        __hip_atomic_store((gu32 *)p.exit_ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

__global__ __launch_bounds__(256, 2) void k44_program_kernel(ProgArgs p) {
    __shared__ ProgLds L;
    if (threadIdx.x == 0u) L.inv_stage = 0u;
    __syncthreads();
    const uint32_t G = gridDim.x, wg = blockIdx.x;
    uint32_t known = 0;
    bool stop = false;
    for (uint32_t s = 0; s < p.nstages && !stop; ++s) {
        const ProgStage st = p.stages[s];
        for (uint32_t i = (wg + G - st.rot % G) % G; i < st.items && !stop; i += G) {
            const uint64_t t_start = p.trace ? wall_clock64() : 0ull;
            switch (st.type) {
            case PROG_WAVES:
                // kreg 2: long contractions, two chunks of one block's A fragments held
                // (plain and 2-operand gathers); otherwise items of prog_bpb blocks
                if (st.prod == 2u) {
                    if (st.kreg > 1u)
                        prog_waves_item<2u, 2u, 1u>(p, st, i, s, known, stop, L);
                    else
                        prog_waves_item<2u, 1u, 2u>(p, st, i, s, known, stop, L);
                } else if (st.prod == 3u) {
                    prog_waves_item<3u, 1u, 1u>(p, st, i, s, known, stop, L);
                } else if (st.prod == 4u) {
                    prog_waves_item<4u, 1u, 2u>(p, st, i, s, known, stop, L);
                } else {
                    if (st.kreg > 1u)
                        prog_waves_item<0u, 2u, 1u>(p, st, i, s, known, stop, L);
                    else
                        prog_waves_item<0u, 1u, 2u>(p, st, i, s, known, stop, L);
                }
                break;
            case PROG_NORM: prog_norm_item(p, p.aux[st.first], i, s, known, stop, L); break;
            case PROG_EMBED: prog_embed_item(p, p.aux[st.first], i, s, known, stop, L); break;
            case PROG_ARGMAX: prog_argmax_item(p, p.aux[st.first], i, s, known, stop, L); break;
            default: prog_argmax_final_item(p, p.aux[st.first], s, known, stop, L); break;
            }
            if (p.trace && threadIdx.x == 0u) {
                uint64_t *r = p.trace + 8ull * (st.base + i);
                r[0] = t_start;
                r[1] = L.t_wait;
                r[2] = wall_clock64();
                r[3] = wg;
                r[4] = st.type == PROG_WAVES ? L.t_mark[0] : 0ull;
                r[5] = st.type == PROG_WAVES ? L.t_mark[1] : 0ull;
                r[6] = L.t_mark[2];
                r[7] = 0ull;
            }
        }
    }
    prog_exit(p, L);
}

hipError_t prog_grid(uint32_t &grid) {
    int dev = 0, cus = 0, occ = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k44_program_kernel, 256, 0);
    if (e != hipSuccess) return e;
    if (occ < 1 || cus < 1) return hipErrorInvalidConfiguration;
    grid = (uint32_t)cus * (uint32_t)(occ < 2 ? occ : 2);
    return hipSuccess;
}

hipError_t launch_program(const ProgArgs &p, uint32_t grid, hipStream_t stream) {
    if (grid == 0u || p.nstages == 0u) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k44_program_kernel, dim3(grid), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace k44dev
