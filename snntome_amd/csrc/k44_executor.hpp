// k44_executor.hpp — the executor of compiled wave plans on MI355X (K44GpuExecutorState), shared
// by its translation units: k44_exec_build.hip (plan validation and upload), k44_exec_schedule.hip
// (fusion, scheduling, the persistent decode program, the report), k44_exec_launch.hip (launches
// and host I/O); k44_wave_executor.hip holds the C ABI over it.
//
// Replaces the reference's K44GpuExecutorState (wavec/k44_wave_executor.cu:76-620).  Design:
//  * One hipMalloc'd fp16 canvas per plan, zeroed at init; all tensors are views into it.
//  * Every K44_WAVE command is turned at upload into a device schedule: the per-synapse index
//    rows are compressed into dendritic segments (start offset, S consecutive positions at a
//    fixed canvas step), the RDNA4-ordered weight blocks are re-laid out into the order the
//    chosen kernel consumes, and every address the kernel can touch is bounds-checked against
//    the canvas on the host before any launch.
//  * Kernels run on a private non-blocking stream (default priority); timing uses HIP events on
//    that stream.
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <memory>
#include <mutex>
#include <numeric>
#include <sstream>

#include "k44_tuning.hpp"
#include "k44_wave_compiler.hpp"
#include "k44wavec.h"
#include "kernels/k44_launch.hpp"
#include "kernels/k44_program.hpp"
#include "kernels/k44_spatial.hpp"

namespace k44_host {
namespace exec {
struct HipFail : std::runtime_error {
    using std::runtime_error::runtime_error;
};

#define K44_HIP(call)                                                                          \
    do {                                                                                       \
        hipError_t e_ = (call);                                                                \
        if (e_ != hipSuccess)                                                                  \
            throw ::k44_host::exec::HipFail(std::string("HIP error '") + hipGetErrorString(e_) + "' in " #call); \
    } while (0)

template <typename T>
struct DevBuf {
    T *p = nullptr;
    size_t n = 0;
    DevBuf() = default;
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    ~DevBuf() { reset(); }
    void reset() {
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
    }
    void alloc(size_t count) {
        reset();
        if (count) K44_HIP(hipMalloc(&p, count * sizeof(T)));
        n = count;
    }
    void upload(const std::vector<T> &h) {
        alloc(h.size());
        if (!h.empty()) K44_HIP(hipMemcpy(p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    }
};

// Device schedule of one K44_WAVE command.
struct WaveExec {
    std::string name;
    std::string path;      // "valu_gather_dot" | "mfma_tile" | "mfma_dma" | "mfma_narrow" | ...
    std::string why;
    bool mfma = false;
    uint32_t mt = 0, rows_per_stage = 32, ksteps = 0;  // MFMA tile: tokens, positions/stage
    uint32_t kgroups = 1, stage_chunk = 0;  // MFMA split-K: workgroups per tile, stages each
    bool narrow = false;       // MFMA over <= 16 tokens (decode): k44_mfma_narrow_kernel
    bool dma = false;          // MFMA over 512-token workgroups: k44_mfma_dma_kernel
    k44dev::DmaShape dshape;   // dma: ring stages, load policy
    bool lane8 = false;        // VALU: 8 tokens (16-byte loads) per lane
    bool stream_loads = false; // VALU: non-temporal X / weight loads (gathered rows >> caches)
    bool stream_kernel = false; // VALU: k44_gather_stream_kernel (output rows staged in LDS)
    bool weights_in_lds = true; // VALU 8-token kernel: neuron weights staged in LDS
    bool misaligned = false;    // segment starts off the 4-element grid (token-shifted taps)
    // MFMA tile kernel over rows off the 16-byte grid (token-shifted taps, single-frame 2-D
    // planes): aligned loads shifted into place before the LDS store (MIS variant)
    bool mis = false;
    bool epi_scalar = false;    // 2-byte epilogue stores (single-frame 2-D tile offsets)
    bool phase_order = false;   // synapses regrouped by token phase (segment_rows)
    uint32_t part_tokens = 0;  // row length of split-K partials (16 narrow, tokens wide)
    uint32_t cout = 0, K = 0, S = 0, cluster = 1, rows = 0;
    uint64_t step = 1;
    uint32_t tokens = 0, out_stride = 0;
    uint32_t slab = 256, U = 4, n_batch = 1, ksplit = 1;
    bool sorted_segments = false;
    uint64_t y_off = 0, res_off = 0;
    int act = 0;
    bool has_res = false;
    double flops = 0.0;          // executed: 2 * Cout * B_raw * tokens (padding included)
    double eff_flops = 0.0;      // 2 * real synapses * valid tokens (the plan's gflops)
    uint64_t unique_rows = 0;    // distinct substrate positions read
    DevBuf<uint64_t> seg;
    DevBuf<__half> w, bias;
    DevBuf<uint16_t> cmap;
    // Canvas element ranges read (gather segments, residual rows) and written (output rows),
    // merged and sorted: the host-side independence test of wave groups.
    std::vector<std::pair<uint64_t, uint64_t>> rd, wr;
    std::vector<std::pair<uint64_t, uint64_t>> xrd, resrd;  // gather segments; residual rows
    // Element-wise multiplies fused into this wave's gather (whole-plan execution only):
    // xprod 2 / 3 leaves at element offsets xd relative to the wave's input tensor; rd_fused =
    // the read ranges of the fused form.
    uint32_t xprod = 0;
    int64_t xd[3] = {0, 0, 0};
    // Whole-plan execution (multiplies folded, operands relocated): output offset and canvas
    // ranges; equal to y_off / rd / wr unless folding changed them.
    uint64_t y_off_run = 0;
    std::vector<std::pair<uint64_t, uint64_t>> rd_run, wr_run;
    size_t part_floats = 0;  // split-K partials (kgroups * cout * tokens), 0 without split-K
    // Narrow 64/128-neuron waves with split-K: whole-plan launches reduce the partials in the
    // last workgroup of each tile (per-tile arrival counters at arrive + arrive_off) instead of
    // a second kernel; command-by-command launches keep the epilogue kernel.
    bool reduce_in_kernel = false;
    bool red_local = false;  // that reduction through one XCD's L2 (MfmaTileArgs::red_local)
    size_t arrive_off = 0;
    // Folded RMSNorm (whole-plan runs): producer of the norm's input (fold index, first slot
    // of this wave's tiles among the fold's tiles), or consumer gathering the normalised rows
    // (xprod 4; the fold whose scales it applies).
    size_t norm_fold = SIZE_MAX;
    uint32_t norm_tile0 = 0;
    size_t xnorm = SIZE_MAX;
    // Narrow waves: segment starts as uploaded ([rows][K], host copy).  Gather form 5 (a folded
    // RMSNorm + decode token shift): per work item the 32-row passes whose channels' shifted
    // state it stores (bit sub-chunk * 16 + pass).  cp_fold: the fold whose state copy this
    // wave's launch carries: the plan's state into the compact copy before the readers
    // (cp_refresh), or the shifted state back into the plan's state after them.
    std::vector<uint64_t> seg_h;
    DevBuf<uint64_t> own;
    size_t cp_fold = SIZE_MAX;
    bool cp_refresh = false;
    // the state range of a carried copy, counted as written when launches are grouped (so the
    // launch never joins one of the fold's readers)
    std::vector<std::pair<uint64_t, uint64_t>> carry_rng;
    // 2-D spatial wave (VALU over the padded-plane tile layout): tile tables, output plane.
    bool tile2d = false;
    DevBuf<uint32_t> tile_x, tile_y;
    k44dev::Plane2D plane{};
    uint32_t tiles = 0, tiles_per_frame = 0;
    int masked = 0;
    // MFMA: descriptor of this wave alone (command-by-command execution).
    DevBuf<k44dev::MfmaTileArgs> one_args;
    DevBuf<uint32_t> one_start;
    k44dev::NarrowPre one_pre;  // narrow kernels: weights and geometry as kernel arguments
    uint32_t items = 0, epi_items = 0;
};

// A launch of several independent MFMA waves of one kernel configuration.
struct MfmaGroupExec {
    std::vector<size_t> members;  // wave indices, plan order
    uint32_t nt = 0, mt = 0, rows = 0, items = 0, epi_items = 0, max_items = 0;
    bool dma = false, stream_loads = false, mis = false;
    uint32_t prod = 0;  // product form (xprod) every member's gathers take
    k44dev::DmaShape dshape;
    size_t part_floats = 0;
    DevBuf<k44dev::MfmaTileArgs> args;
    DevBuf<uint32_t> start;
    k44dev::NarrowPre pre;  // narrow kernels: up to six members' weights and geometry
    DevBuf<__half> pre_w;   // those members' A fragments, member m at (m << pre.shift) bytes
};

// Sorted, merged [lo, hi) element ranges.
using Ranges = std::vector<std::pair<uint64_t, uint64_t>>;

inline Ranges merge_ranges(Ranges r) {
    std::sort(r.begin(), r.end());
    Ranges out;
    for (const auto &x : r) {
        if (!out.empty() && x.first <= out.back().second)
            out.back().second = std::max(out.back().second, x.second);
        else
            out.push_back(x);
    }
    return out;
}

inline bool ranges_overlap(const Ranges &a, const Ranges &b) {
    size_t i = 0, j = 0;
    while (i < a.size() && j < b.size()) {
        if (a[i].second <= b[j].first)
            ++i;
        else if (b[j].second <= a[i].first)
            ++j;
        else
            return true;
    }
    return false;
}

// Device schedule of one 1-D token op (RMSNORM_1D, SWIGLU_MUL_1D, TOKEN_SHIFT_1D, EMBED_1D,
// ARGMAX_1D).
struct AuxExec {
    k44_host::K44CmdType type;
    std::string name;
    uint64_t y_off = 0, src_off = 0, src2_off = 0, state_off = 0;
    uint32_t D = 0, stride = 0, tokens = 0, rf = 0, seq_len = 0, vocab = 0;
    bool decode = false, has_state = false;
    bool fused = false;  // SWIGLU_MUL_1D folded into its consumers' gathers, or TOKEN_SHIFT_1D
                         // run by the RMSNorm before it (not launched)
    size_t shift_with = SIZE_MAX;  // RMSNORM_1D: the decode token shift it runs (whole plans)
    size_t norm_fold = SIZE_MAX;   // RMSNORM_1D: its scales come from the producers' sums
    // EMBED_1D (decode): the fold whose producer it is (it stores the sums of squares of its
    // 64-channel blocks from slot slot_tile0 of the fold on)
    size_t slot_fold = SIZE_MAX;
    uint32_t slot_tile0 = 0;
    // EMBED_1D (decode, whole-plan runs): the fold whose compact token-shift state copy this
    // launch refreshes from the plan's state (the first layer's readers have no narrow launch
    // before them to do it)
    size_t cp_fold = SIZE_MAX;
    // SWIGLU_MUL_1D y = other * q where q = b * c is an inner multiply only this one reads:
    // whole plans run both as y = fp16(other * fp16(b * c)) (the inner one is not launched).
    size_t chain_inner = SIZE_MAX;
    uint64_t chain_other = 0;
    std::string fuse_note;         // SWIGLU_MUL_1D: why it was or was not folded (report)
    float eps = 1e-5f;
    DevBuf<__half> table;  // gamma (RMSNORM), mix (TOKEN_SHIFT), embedding table (EMBED)
    // 2-D spatial commands (S2D, pools, upsample, scatter-upconv): channel count C, planes
    k44dev::Plane2D pin{}, pout{};
    uint32_t C = 0, out_channels = 0;
};

inline k44dev::Plane2D plane_of(const k44_host::K44ResDesc &L) {
    return k44dev::Plane2D{L.H, L.W, L.W_pad, L.batch_size, L.single_stride, L.channel_stride,
                           L.is_image_token64 ? 1u : 0u};
}

// Canvas elements allocated past the plan's canvas: the misaligned 2-D gathers read up to 3
// elements beyond the last one they use.
inline constexpr uint64_t kCanvasSlack = 256;

// Tokens per MFMA workgroup: the widest tile that divides the token count (most reuse of each
// weight fragment; a 64-token workgroup is one wave with a long serial loop, measured slower
// than a wider tile plus split-K on the same wave).
inline uint32_t pick_mt(uint32_t tokens) {
    for (uint32_t mt : {512u, 256u, 128u}) if (tokens % mt == 0u) return mt;
    return 64u;
}

inline uint32_t pick_slab(uint32_t tokens) {
    if (tokens % 256u == 0u) return 256u;
    if (tokens % 128u == 0u) return 128u;
    return 64u;
}

}  // namespace exec

using namespace exec;

struct K44GpuExecutorState {
    K44WavePlan plan_meta;  // plan without payload vectors
    std::vector<std::unique_ptr<WaveExec>> waves;
    std::vector<std::unique_ptr<AuxExec>> aux;
    // Plan commands in order: (is_wave, index); the plan runs as `runs`: an aux command, a VALU
    // wave, or a group of independent MFMA waves (kind 0 / 1 / 2, index).
    std::vector<std::pair<bool, size_t>> ops;
    std::vector<std::pair<int, size_t>> runs;
    std::vector<size_t> wave_cmd, aux_cmd;  // plan command index of every wave / aux command
    std::vector<std::unique_ptr<MfmaGroupExec>> groups;
    DevBuf<__half> canvas;
    DevBuf<uint32_t> ids, history, step_ctr;  // token ids (EMBED / ARGMAX), greedy history
    DevBuf<uint16_t> stage;  // packed strided canvas reads (wavec_gpu_read_canvas_2d)
    uint32_t id_tokens = 0, hist_steps = 0;
    // Scratch shared by the commands of the plan (they run in order on one stream): split-K
    // partials of MFMA waves, per-chunk (value, index) partials of ARGMAX.
    DevBuf<float> scratch;
    size_t scratch_need = 0;  // floats
    // Per-tile arrival counters of the waves that reduce split-K in the launch (zeroed at init;
    // each launch leaves them at zero).
    DevBuf<uint32_t> arrive;
    // XCD-local split-K meetings: set-up found workgroups 8 apart in launch order sharing an
    // XCD; any_local: some wave meets that way (its counters are checked after each run).
    bool xcd_local_ok = false, any_local = false;
    size_t n_arrive = 0;
    // Folded RMSNorms (fuse_norms): per fold the producers' tile slots (16 tokens x 4 words
    // each: the exact sums of squares of the values the tile stored).
    struct NormFold {
        size_t norm = 0;            // aux index of the RMSNORM_1D command
        uint32_t tiles = 0;         // producer tiles (slots)
        size_t slot0 = 0;           // first slot in norm_slots
        bool consumers = false;     // not launched: its readers gather normalised rows
        // The decode token shift run with the norm (its readers gather shifted rows, gather
        // form 5), and the fold's regions of shift_next ([D][rf-1][16] each): the shifted
        // state (next0) and the compact copy of the state its readers read (cur0).
        size_t shift = SIZE_MAX;
        size_t next0 = 0, cur0 = 0;
        size_t mix0 = 0;  // its [D][8] table in shift_mix (MfmaTileArgs::mixg)
    };
    std::vector<NormFold> norm_folds;
    DevBuf<uint32_t> norm_slots;
    DevBuf<__half> shift_next, shift_mix;
    size_t shift_next_elems = 0;
    const uint64_t *fold_slots(size_t fold) const {
        return reinterpret_cast<const uint64_t *>(norm_slots.p + norm_folds[fold].slot0 * 64u);
    }
    uint64_t fold_elems = 0;  // private region past the canvas for relocated multiply operands
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    bool use_graph = false;
    bool initialized = false;
    uint32_t xcd_order = 2;  // MFMA tile kernels: item order over the XCDs (MfmaGroup)
    std::string report_json;
    // Decode-sized plans whose runs are all narrow projections, decode RMSNorms (with their
    // token shifts), embeddings and argmaxes run whole-plan executions as one persistent launch
    // (kernels/k44_program.hpp); `prog_why` says why a plan does not.
    bool prog_active = false;
    std::string prog_why = "not built";
    uint32_t prog_grid = 0;
    std::vector<k44dev::ProgStage> prog_stages_h;
    DevBuf<k44dev::ProgStage> prog_stages;
    DevBuf<k44dev::ProgWave> prog_waves;
    DevBuf<k44dev::ProgAux> prog_aux;
    DevBuf<uint32_t> prog_ctrs;  // [nstages] completion counters, exit counter, abort word
    DevBuf<uint64_t> prog_zero;  // 64 argmax keys (zero between launches)
    DevBuf<uint64_t> prog_slots; // folded RMSNorms: per producer item 16 tokens x 2 sum words
    DevBuf<__half> prog_shadow;  // per stage the span of canvas it writes (read by later stages)
    DevBuf<uint64_t> prog_trace; // tuning prog_trace=1: 8 words per item of the last launch
    k44dev::ProgArgs prog_args{};


    ~K44GpuExecutorState() { free_all(); }

    const K44ResDesc &layout(uint32_t key) const { return plan_meta.res_map.at(key); }

    // Plan validation and device upload (k44_exec_build.hip): index rows to segment
    // schedules, kernel and split choice per wave, weight re-layout, bounds checks, descriptors.
    void free_all();
    void drop_graph();
    static void segment_rows(const K44ExecCmd &c, uint64_t step, uint32_t &S_out,
                             std::vector<uint64_t> &starts, std::vector<uint32_t> &perm,
                             bool reorder);
    static bool streaming_gather(const WaveExec &wx);
    void configure_mfma(const K44ExecCmd &c, WaveExec &wx, const std::vector<uint16_t> &wraw,
                        size_t rows, uint32_t width);
    void build_wave(const K44ExecCmd &c, WaveExec &wx);
    void build_wave2d(const K44ExecCmd &c, WaveExec &wx, const K44ResDesc &Lo,
                      const K44ResDesc &Li);
    void build_spatial(const K44ExecCmd &c, AuxExec &ax);
    void build_aux(const K44ExecCmd &c, AuxExec &ax);
    void init(const K44WavePlan &plan);
    static void set_split(WaveExec &w, uint32_t want);
    k44dev::MfmaTileArgs mfma_args(const WaveExec &w, float *part, bool fused) const;
    static uint32_t epi_workgroups(const WaveExec &w);
    void upload_mfma_descriptors();
    static uint32_t item_stages(const WaveExec &w);
    k44dev::NarrowPre narrow_pre(const std::vector<k44dev::MfmaTileArgs> &args,
                                 const std::vector<size_t> &members, DevBuf<__half> *arena);
    void probe_xcd_placement();
    void check_placement();
    static void check_balanced_order(const std::vector<uint32_t> &start);

    // Fusion and scheduling (k44_exec_schedule.hip): folded multiplies and RMSNorms, the
    // runs of a whole-plan execution and their group launches, the persistent decode program,
    // the execution report.
    void aux_ranges(const AuxExec &a, Ranges &rd, Ranges &wr) const;
    void fuse_products();
    void fuse_mul_chains();
    void fuse_norm_shifts();
    bool fold_shift(size_t i, const std::pair<uint64_t, uint64_t> &X,
                    const std::pair<uint64_t, uint64_t> &Y, const std::vector<Ranges> &rd,
                    const std::vector<Ranges> &wr, const Ranges &out_rng,
                    std::vector<size_t> &cons, size_t &refresher, size_t &carrier,
                    std::vector<std::vector<uint64_t>> &owns, size_t embed_aux);

    void fuse_norms();
    void form_runs();
    size_t launches_per_run() const;
    void build_report();
    void drop_program(const std::string &why);
    void build_program();
    void check_program();

    // Launches and host I/O (k44_exec_launch.hip).
    void launch_aux(const AuxExec &a, bool whole = false);
    void launch_mfma_group(const k44dev::MfmaGroup &d, uint32_t nt, uint32_t mt, uint32_t rows,
                           uint32_t items, uint32_t epi_items, bool dma, const k44dev::DmaShape &ds,
                           uint32_t prod, uint32_t max_items, bool mis,
                           const k44dev::NarrowPre &pre);
    void launch_mfma(const WaveExec &w);
    void launch_group(const MfmaGroupExec &g);
    void launch_wave(const WaveExec &w);
    void launch_op(size_t i);
    void launch_ops(size_t first = 0, size_t n = SIZE_MAX);
    void execute_plan();
    void set_history(uint32_t steps);
    void upload_input_f32(const float *in, size_t n);
    std::vector<float> download_output_f32();
    int infer_f32(const float *in, int in_elems, float *out, int out_elems, float *ms_out);
};

}  // namespace k44_host
