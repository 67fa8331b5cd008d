// k44_tuning.hpp — process-wide tuning switches of the wave executor.
//
// Every switch defaults to -1: the executor decides from the plan (the measured defaults
// documented where each decision is made).  Tests and benchmarks force a choice through
// wavec_set_tuning(key, value) to compare paths that must give identical or tolerance-equal
// results; the value is read when a plan is initialised (wavec_gpu_init_plan), so a plan keeps
// the choices it was built with.  No switch changes a plan's semantics, only how it is run.
#pragma once

namespace k44_host {

enum class Tune : int {
    Path = 0,      // "path":          0 VALU gather-dot for every wave, 1 MFMA where it applies
    Dma,           // "dma":           0 = register-staged MFMA tile instead of the LDS ring
    DmaStages,     // "dma_stages":    2 or 4 LDS ring stages
    NonTemporal,   // "nt":            0 / 1 non-temporal gather loads
    SplitK,        // "splitk":        0 = no split-K on wide MFMA waves
    Lane8,         // "lane8":         0 / 1 eight tokens per lane in the VALU kernels
    KSplit,        // "ksplit":        1 or 4 waves per neuron in the VALU kernel
    StreamKernel,  // "stream_kernel": 0 / 1 streaming VALU kernel (output rows staged in LDS)
    Narrow,        // "narrow":        0 = no narrow (<= 16 token) MFMA kernel
    NarrowChunk,   // "narrow_chunk":  longest contraction chunk of the narrow kernel, >= 16 k-steps
    Group,         // "group":         0 = every MFMA wave launched alone
    GroupSplit,    // "group_split":   0 = group launches keep their members' split-K
    Fuse,          // "fuse":          0 = no folded multiplies / RMSNorm+token-shift kernels
    SortSegments,  // "sort":          0 = segments in index-row order (not address order)
    WeightsInLds,  // "wlds":          0 = 8-token VALU kernel reads weights per batch
    Token64Ring,   // "t64_ring":      0 per-wave Token64 kernel, 1 / 2 64- / 128-neuron ring kernel
    XcdOrder,      // "xcd_order":     0 = MFMA tile kernels take items in workgroup order,
                   //                  1 = contiguous item ranges per XCD, 2 = per-wave shares
    NarrowWgs,     // "narrow_wgs":    workgroups a narrow wave of >= 64-neuron tiles is split to
                   //                  reach (>= 1; contraction chunks of >= 16 k-steps)
    NarrowReduce,  // "narrow_reduce": 0 = split narrow waves reduce in k44_splitk_epilogue_kernel,
                   //                  1 = the last workgroup of each tile reduces in the launch
    DmaProd,       // "dma_prod":      0 = LDS-ring MFMA waves load and multiply in every wave,
                   //                  1 = producer waves issue the loads (4-stage ring)
    Program,       // "program":       1 = decode-sized plans run each whole-plan execution as one
                   //                  persistent launch (k44_program.hpp); automatic and 0:
                   //                  kernel by kernel (measured faster on config-5 decode)
    ProgSpinMs,    // "prog_spin_ms":  wait limit of the persistent launch's stage waits (ms, >= 0;
                   //                  automatic: 1000), past which the launch is abandoned
    ProgTrace,     // "prog_trace":    1 = the persistent launch records per-item timestamps
                   //                  (wavec_gpu_program_trace)
    NarrowPre,     // "narrow_pre":    0 = narrow waves read their weights' address and geometry
                   //                  from their descriptors; automatic and 1: up to six waves
                   //                  of a launch take them as preloaded kernel arguments
    NarrowLocal,   // "narrow_local":  0 = split narrow waves reduced in the launch meet through
                   //                  device-coherent memory; automatic and 1: through the L2 of
                   //                  the XCD all chunks of a tile run on (items renumbered so
                   //                  they are 8 workgroups apart), where set-up finds that
                   //                  workgroups 8 apart share an XCD
    EmbedRefresh,  // "embed_refresh": 0 = a decode embedding never refreshes a folded token
                   //                  shift's state copy (the first layer's RMSNorm + shift then
                   //                  runs as its own kernel); automatic and 1: it does
    NarrowByy,     // "narrow_byy":    0 = narrow group launches find each workgroup's wave in the
                   //                  group's prefix sums; automatic: (workgroups x waves) grids
                   //                  where they launch at most 1.5x the work items
    Count
};

// Current value of a switch (-1 = automatic).
int tune(Tune t);

}  // namespace k44_host
