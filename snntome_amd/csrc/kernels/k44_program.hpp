// k44_program.hpp — a decode-sized plan run as one launch of a persistent kernel.
//
// A decode step is a chain of ~80 small dependent operations (embedding, per layer an RMSNorm
// with its token shift and four narrow projections, the head, argmax).  Launched one kernel per
// operation, every link pays a launch, the first round trip of its weight stream, and (for the
// projections split over the chip) a cross-workgroup reduction: the step is latency-bound at a
// few percent of HBM bandwidth although its weights are only ~1 GB.
//
// Here the plan's runs become the stages of one program, executed by a grid that is resident
// all at once (occupancy x compute units, checked on the host).  Stage s has `items` work items;
// item i runs on workgroup (i + rot) % G.  An item that reads what earlier stages wrote first
// issues its loads of read-only data (weights, gammas, mixing weights, its own state rows), then
// waits until stage s - 1 has signalled completion of every item (a device-scope counter), then
// reads its inputs and signals stage s.  Stage s - 1 complete implies every earlier stage is
// complete (each of its items waited for s - 2 before signalling), so one counter per stage
// orders every read-after-write and write-after-read hazard of the plan.  The weight stream of
// the next projection thus runs while the previous one finishes.
//
// Projections run as 16-neuron x whole-contraction items: the 4 waves of the workgroup take a
// quarter of the k-steps each (A fragments held in registers, requested before the wait) and
// meet in LDS in wave order.  No item needs another workgroup's partial sums.
//
// Coherence without cache write-backs: every store of the program is device-coherent
// (agent-scope relaxed atomic stores, not left dirty in an XCD's L2), and each wave waits for
// its stores (vmcnt 0) before the barrier that precedes the completion signal.  Reads go
// through the caches: a stage writes its outputs twice, to the canvas (what the host and the
// next launch see) and to a shadow region of its own that nothing else writes, and later
// stages read the shadow of the stage that produced their input.  A shadow line is written
// once per launch and read only after that write, and every launch starts with the caches
// invalidated, so no XCD can hold an older copy of it (the canvas itself may reuse a line for
// several tensors in one launch).  Read-only data (weights, tables, segment starts) and the
// norm slots below (also written once per launch) are read the same way.
//
// RMSNorm sums of squares are exact integers (k44_sumsq.hpp): every producer item stores the
// sums of the values it stored in its own slot, and each consuming workgroup adds all slots
// (any order gives the same integer, so the scales are the norm kernel's bits) once per stage.
// Argmax keys (orderable value, inverted channel) meet in 64-bit atomic maxima, also
// order-independent.
// The program is therefore deterministic: eager launches and graph replays agree bit for bit.
//
// Waits are bounded: a wait that exceeds `spin_ticks` of the 100 MHz real-time counter sets
// `abort`, every other wait sees it, every workgroup skips its remaining items and exits, and
// the host reports the stage.  The last workgroup to exit returns the counters, sums and keys
// to zero for the next launch.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace k44dev {

enum ProgStageType : uint32_t {
    PROG_WAVES = 0,         // narrow projections (16-neuron x whole-contraction items)
    PROG_NORM = 1,          // decode RMSNorm (+ decode token shift), 128-channel items
    PROG_EMBED = 2,         // embedding rows of the token ids, 128-channel items
    PROG_ARGMAX = 3,        // per-token maxima of 128-channel blocks into 64-bit keys
    PROG_ARGMAX_FINAL = 4,  // keys -> ids (+ greedy history), one item
};

struct ProgStage {
    uint32_t type;
    uint32_t items;  // work items (each signals completion once)
    uint32_t first;  // PROG_WAVES: first ProgWave of the stage; otherwise the ProgAux
    uint32_t count;  // PROG_WAVES: waves of the stage
    uint32_t rot;    // item i runs on workgroup (i + rot) % G
    uint32_t prod;   // PROG_WAVES: gather form of the stage's waves (0, 2, 3, 4)
    uint32_t kreg;   // PROG_WAVES: 8-k-step chunks of A fragments held per wave (1 or 2)
    uint32_t base;   // items of the stages before this one (trace record index)
};

// One narrow wave (NT-neuron tiles sharing an index row; NT = 16 * nb).
struct ProgWave {
    // Gather operand bases: element e of operand k is Xo[k][e] for the canvas element offsets e
    // of the segment rows (the producing stage's shadow, or the canvas, with the operand's
    // offset from the segment rows folded in).
    const __half *Xo[3];
    const uint64_t *seg;    // [tiles][K] canvas element offset of each segment start
    const __half *Wf;       // [tile][k-step][nb][64 lanes][8] A fragments
    const __half *bias;     // [cout] or nullptr
    const uint16_t *cmap;   // [cout] output row of each neuron (0xffff: empty slot) or nullptr
    __half *Y;              // output base (canvas)
    __half *Ys;             // output base in this stage's shadow
    const __half *R;        // residual base (producer's shadow or canvas) or nullptr
    const __half *xgamma;   // gather form 4: RMSNorm gamma (nullptr: 1)
    // Folded RMSNorm, producer side: per item of the stage 16 tokens x 2 words (limbs 0 | 1,
    // limb 2 | inf / NaN flags) of the exact sums of squares of the values it stored, at
    // slot_out + 32 * (item index in the stage); nullptr: none.
    uint64_t *slot_out;
    // Consumer side (gather form 4): the slot_n item slots of the norm's producers.
    const uint64_t *slot_in;
    uint64_t step;          // canvas elements between consecutive positions of a segment
    uint64_t xg_base;       // gather form 4: gamma row = (row offset - xg_base) >> xg_shift
    uint32_t K, S, ksteps, nb, tiles;
    uint32_t item0;         // first item of this wave within its stage (items: tile * nb + block)
    uint32_t out_stride;
    int act;
    uint32_t xg_shift, norm_D;
    float norm_eps;
    uint32_t slot_n;
};

// RMSNorm (+ decode token shift), embedding, argmax.
struct ProgAux {
    __half *y, *ys;          // NORM / EMBED output: canvas, this stage's shadow
    const __half *x;         // NORM input, ARGMAX logits (producer's shadow or canvas)
    const __half *table;     // NORM gamma (nullptr: 1), EMBED table
    __half *y2, *y2s;        // NORM: token-shift output (nullptr: no shift), and its shadow
    const __half *mu;        // NORM: mixing weights [D][rf]
    __half *state;           // NORM: shift state [D][rf - 1][64] (nullptr when rf == 1)
    const uint64_t *slot_in; // NORM: x's producers' item slots (as ProgWave; nullptr: summed here)
    uint64_t *keys;          // ARGMAX / ARGMAX_FINAL: [64] per-token keys
    const uint32_t *ids_in;  // EMBED
    uint32_t *ids_out;       // ARGMAX_FINAL
    uint32_t *history;       // ARGMAX_FINAL: [hist_steps][tokens] or nullptr
    uint32_t *step_ctr;      // ARGMAX_FINAL
    uint32_t D, stride, tokens, rf, vocab, hist_steps;
    float eps;
    uint32_t slot_n;
};

struct ProgArgs {
    const ProgStage *stages;
    const ProgWave *waves;
    const ProgAux *aux;
    uint32_t *done;       // [nstages] completion counters (zero between launches)
    uint32_t *exit_ctr;   // workgroups that have exited (zero between launches)
    uint32_t *abort;      // 0, or 1 + the stage whose wait timed out (cleared by the host)
    uint64_t *zero_base;  // argmax keys: zeroed by the last workgroup
    uint64_t spin_ticks;  // wait limit (100 MHz real-time counter ticks)
    // nullptr, or per item (stage base + item) 8 words: real-time counter at the item start,
    // its wait released, its completion signalled; the workgroup that ran it; projection items
    // also when their first inputs arrived and their MFMAs were done; any item when its
    // stores were performed
    uint64_t *trace;
    uint32_t nstages, zero_words;
};

// 16-neuron blocks per projection item: 2, except for long contractions (kreg 2: one block,
// two chunks of its A fragments held) and 3-operand gathers (their rows take the registers).
inline uint32_t prog_bpb(uint32_t prod, uint32_t kreg) { return (kreg > 1u || prod == 3u) ? 1u : 2u; }

// Items per 128-channel stage.
inline uint32_t prog_channel_items(uint32_t D) { return (D + 127u) / 128u; }

// The kernel's resident grid: occupancy (workgroups per compute unit, at most 2) x units.
hipError_t prog_grid(uint32_t &grid);
hipError_t launch_program(const ProgArgs &p, uint32_t grid, hipStream_t stream);

}  // namespace k44dev
