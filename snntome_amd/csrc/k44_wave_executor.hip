// k44_wave_executor.hip — MI355X executor for compiled wave plans + the wavec C ABI.
//
// Replaces the reference's wavec/k44_wave_executor.cu (K44GpuExecutorState and the extern "C"
// frontend at :642-988).  The C ABI keeps the reference's 30 entry points with the same
// signatures, argument meaning and 0 / -1 return convention, and adds the build extensions
// declared in include/k44wavec.h.
//
// Executor design (gfx950):
//  * One hipMalloc'd fp16 canvas per plan, zeroed at init; all tensors are views into it.
//  * Every K44_WAVE command is turned at upload into a device schedule: the per-synapse index
//    rows are compressed into dendritic segments (start offset, S consecutive positions at a
//    fixed canvas step), the RDNA4-ordered weight blocks are re-laid out into the order the
//    chosen kernel consumes, and every address the kernel can touch is bounds-checked against
//    the canvas on the host before any launch.
//  * Kernels run on a private non-blocking stream (default priority); timing uses HIP events on
//    that stream.
//  * Errors never terminate the process: each entry point returns -1 and records a message
//    readable through wavec_last_error().
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

namespace {
// Switch values (-1 = automatic) and their wavec_set_tuning keys, in Tune order.
std::atomic<int> g_tune[(int)Tune::Count];
const char *const kTuneKeys[(int)Tune::Count] = {
    "path", "dma", "dma_stages", "nt", "splitk", "lane8", "ksplit", "stream_kernel", "narrow",
    "narrow_chunk", "group", "group_split", "fuse", "sort", "wlds", "t64_ring", "xcd_order",
    "narrow_wgs", "narrow_reduce", "dma_prod", "program", "prog_spin_ms", "prog_trace"};
// Values each switch honours besides -1: a set of small values (bit v of `set`), or every
// value >= `min` when `set` is 0.  Anything else is refused, so an A/B run cannot measure a
// configuration other than the one it asked for.
struct TuneValues {
    uint32_t set;
    int min;
};
constexpr uint32_t V01 = 0x3u;
const TuneValues kTuneValues[(int)Tune::Count] = {
    {V01, 0},          // path 0 | 1
    {V01, 0},          // dma
    {0x14u, 0},        // dma_stages 2 | 4
    {V01, 0},          // nt
    {V01, 0},          // splitk
    {V01, 0},          // lane8
    {0x12u, 0},        // ksplit 1 | 4
    {V01, 0},          // stream_kernel
    {V01, 0},          // narrow
    {0u, 16},          // narrow_chunk >= 16
    {V01, 0},          // group
    {V01, 0},          // group_split
    {V01, 0},          // fuse
    {V01, 0},          // sort
    {V01, 0},          // wlds
    {0x7u, 0},         // t64_ring 0 | 1 | 2
    {0x7u, 0},         // xcd_order 0 | 1 | 2
    {0u, 1},           // narrow_wgs >= 1
    {V01, 0},          // narrow_reduce
    {V01, 0},          // dma_prod
    {V01, 0},          // program
    {0u, 0},           // prog_spin_ms >= 0
    {V01, 0},          // prog_trace
};
struct TuneInit {
    TuneInit() {
        for (auto &v : g_tune) v.store(-1);
    }
} g_tune_init;
}  // namespace

int tune(Tune t) { return g_tune[(int)t].load(std::memory_order_relaxed); }

}  // namespace k44_host

namespace {

thread_local std::string g_last_error;

void set_error(const std::string &m) {
    g_last_error = m;
    std::fprintf(stderr, "[k44wavec] %s\n", m.c_str());
}

struct HipFail : std::runtime_error {
    using std::runtime_error::runtime_error;
};

#define K44_HIP(call)                                                                          \
    do {                                                                                       \
        hipError_t e_ = (call);                                                                \
        if (e_ != hipSuccess)                                                                  \
            throw HipFail(std::string("HIP error '") + hipGetErrorString(e_) + "' in " #call); \
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
    size_t arrive_off = 0;
    // Folded RMSNorm (whole-plan runs): producer of the norm's input (fold index, first slot
    // of this wave's tiles among the fold's tiles), or consumer gathering the normalised rows
    // (xprod 4; the fold whose scales it applies).
    size_t norm_fold = SIZE_MAX;
    uint32_t norm_tile0 = 0;
    size_t xnorm = SIZE_MAX;
    // 2-D spatial wave (VALU over the padded-plane tile layout): tile tables, output plane.
    bool tile2d = false;
    DevBuf<uint32_t> tile_x, tile_y;
    k44dev::Plane2D plane{};
    uint32_t tiles = 0, tiles_per_frame = 0;
    int masked = 0;
    // MFMA: descriptor of this wave alone (command-by-command execution).
    DevBuf<k44dev::MfmaTileArgs> one_args;
    DevBuf<uint32_t> one_start;
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
};

// Sorted, merged [lo, hi) element ranges.
using Ranges = std::vector<std::pair<uint64_t, uint64_t>>;

Ranges merge_ranges(Ranges r) {
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

bool ranges_overlap(const Ranges &a, const Ranges &b) {
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

k44dev::Plane2D plane_of(const k44_host::K44ResDesc &L) {
    return k44dev::Plane2D{L.H, L.W, L.W_pad, L.batch_size, L.single_stride, L.channel_stride,
                           L.is_image_token64 ? 1u : 0u};
}

// Canvas elements allocated past the plan's canvas: the misaligned 2-D gathers read up to 3
// elements beyond the last one they use.
constexpr uint64_t kCanvasSlack = 256;

// Tokens per MFMA workgroup: the widest tile that divides the token count (most reuse of each
// weight fragment; a 64-token workgroup is one wave with a long serial loop, measured slower
// than a wider tile plus split-K on the same wave).
uint32_t pick_mt(uint32_t tokens) {
    for (uint32_t mt : {512u, 256u, 128u}) if (tokens % mt == 0u) return mt;
    return 64u;
}

uint32_t pick_slab(uint32_t tokens) {
    if (tokens % 256u == 0u) return 256u;
    if (tokens % 128u == 0u) return 128u;
    return 64u;
}

}  // namespace

namespace k44_host {

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
    // Folded RMSNorms (fuse_norms): per fold the producers' tile slots (16 tokens x 4 words
    // each), a tile counter (zero between launches) and 64 per-token scales.
    struct NormFold {
        size_t norm = 0;            // aux index of the RMSNORM_1D command
        uint32_t tiles = 0;         // producer tiles (slots)
        size_t slot0 = 0;           // first slot in norm_slots
        bool consumers = false;     // not launched: its readers gather normalised rows
    };
    std::vector<NormFold> norm_folds;
    DevBuf<uint32_t> norm_slots, norm_ctrs;
    DevBuf<float> norm_invs;
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
    DevBuf<uint64_t> prog_trace; // tuning prog_trace=1: 4 words per item of the last launch
    k44dev::ProgArgs prog_args{};

    ~K44GpuExecutorState() { free_all(); }

    void drop_graph() {
        if (graph_exec) (void)hipGraphExecDestroy(graph_exec);
        if (graph) (void)hipGraphDestroy(graph);
        graph_exec = nullptr;
        graph = nullptr;
    }

    void drop_program(const std::string &why) {
        prog_active = false;
        prog_why = why;
        prog_grid = 0;
        prog_stages_h.clear();
        prog_stages.reset();
        prog_waves.reset();
        prog_aux.reset();
        prog_ctrs.reset();
        prog_zero.reset();
        prog_slots.reset();
        prog_shadow.reset();
        prog_trace.reset();
        prog_args = k44dev::ProgArgs{};
    }

    // The persistent decode program of a whole-plan run (kernels/k44_program.hpp), when every
    // run is one of: a launch of narrow 64 / 128-neuron MFMA waves (<= 16 tokens, gather forms
    // 0 / 2 / 3 / 4, 4-element aligned outputs and residuals), a decode RMSNorm with or without
    // its decode token shift (rf <= 5), an embedding, an argmax.  Runs become stages in plan
    // order; folded RMSNorms keep their producers and consumers: the producing launch's items
    // store their sums of squares in slots, and the consumers add the slots.
    void build_program() {
        drop_program("not built");
        if (tune(Tune::Program) != 1) {
            // config-5 decode measured 1.54 ms per step as one persistent launch against 0.85
            // kernel by kernel: each stage waits for its slowest item, whose stores and
            // completion signal queue behind the other workgroups' weight prefetches
            prog_why = "off (kernel-by-kernel launches measured faster; tuning program=1 builds it)";
            return;
        }
        const size_t nfold = norm_folds.size();
        // the stage whose items produce each folded norm's input (all its waves, one stage)
        std::vector<size_t> fold_stage(nfold, SIZE_MAX);
        std::vector<size_t> aux_fold;  // per ProgAux: the fold of a NORM run with its scales
        std::vector<size_t> wave_fold_in;  // per ProgWave: the fold a gather form 4 applies
        std::vector<size_t> prog_wave_src;  // per ProgWave: its WaveExec
        // Shadows: canvas ranges each stage writes; per ProgWave its gather operands' and
        // residual's canvas ranges, per ProgAux the range it reads (resolved to the shadow of
        // the stage that wrote them last, or the canvas).
        std::vector<Ranges> st_wr;
        std::vector<std::vector<Ranges>> pw_ops;
        std::vector<Ranges> pw_res;
        std::vector<Ranges> pa_rd;
        std::vector<k44dev::ProgStage> st;
        std::vector<k44dev::ProgWave> pw;
        std::vector<k44dev::ProgAux> pa;
        auto fail = [&](const std::string &why) {
            prog_why = why;
            return;
        };
        auto al = [](uint64_t off, uint64_t m) { return off % m == 0u; };
        bool has_argmax = false;
        for (const auto &r : runs) {
            k44dev::ProgStage g{};
            if (r.first == 0) {
                const AuxExec &A = *aux[r.second];
                k44dev::ProgAux x{};
                Ranges rdr, wrr;
                x.D = A.D;
                x.stride = A.stride;
                x.tokens = A.tokens;
                x.eps = A.eps;
                if (A.stride != 64u || A.tokens == 0u || A.tokens > 16u)
                    return fail("command '" + A.name + "' is not decode-sized");
                switch (A.type) {
                case K44CmdType::RMSNORM_1D: {
                    if (!al(A.src_off, 8u) || !al(A.y_off, 8u))
                        return fail("RMSNorm '" + A.name + "' rows are not 16-byte aligned");
                    x.y = canvas.p + A.y_off;
                    x.x = canvas.p + A.src_off;
                    x.table = A.table.p;
                    rdr = {{A.src_off, A.src_off + (uint64_t)A.D * A.stride}};
                    wrr = {{A.y_off, A.y_off + (uint64_t)A.D * A.stride}};
                    if (A.shift_with != SIZE_MAX) {
                        const AuxExec &T = *aux[A.shift_with];
                        if (!T.decode || T.rf == 0u || T.rf > 5u || (T.rf > 1u && !T.has_state) ||
                            !al(T.y_off, 8u) || (T.has_state && !al(T.state_off, 8u)))
                            return fail("token shift '" + T.name + "' has no program form");
                        x.y2 = canvas.p + T.y_off;
                        wrr.push_back({T.y_off, T.y_off + (uint64_t)T.D * T.stride});
                        x.mu = T.table.p;
                        x.state = T.has_state ? canvas.p + T.state_off : nullptr;
                        x.rf = T.rf;
                    }
                    g.type = k44dev::PROG_NORM;
                    g.items = k44dev::prog_channel_items(A.D);
                    break;
                }
                case K44CmdType::EMBED_1D:
                    if (A.D % 8u != 0u || !al(A.y_off, 8u) || !ids.p)
                        return fail("embedding '" + A.name + "' has no program form");
                    x.y = canvas.p + A.y_off;
                    x.table = A.table.p;
                    x.ids_in = ids.p;
                    wrr = {{A.y_off, A.y_off + (uint64_t)A.D * A.stride}};
                    x.vocab = A.vocab;
                    g.type = k44dev::PROG_EMBED;
                    g.items = k44dev::prog_channel_items(A.D);
                    break;
                case K44CmdType::ARGMAX_1D:
                    if (!al(A.src_off, 8u) || has_argmax || !ids.p)
                        return fail("argmax '" + A.name + "' has no program form");
                    has_argmax = true;
                    x.x = canvas.p + A.src_off;
                    x.ids_out = ids.p;
                    rdr = {{A.src_off, A.src_off + (uint64_t)A.D * A.stride}};
                    x.history = hist_steps ? history.p : nullptr;
                    x.step_ctr = step_ctr.p;
                    x.hist_steps = hist_steps;
                    g.type = k44dev::PROG_ARGMAX;
                    g.items = k44dev::prog_channel_items(A.D);
                    break;
                default:
                    return fail("command '" + A.name + "' (" + cmd_type_str(A.type) +
                                ") has no program form");
                }
                g.first = (uint32_t)pa.size();
                g.count = 1u;
                aux_fold.push_back(A.type == K44CmdType::RMSNORM_1D ? A.norm_fold : SIZE_MAX);
                pa.push_back(x);
                pa_rd.push_back(rdr);
                st.push_back(g);
                st_wr.push_back(merge_ranges(wrr));
                if (A.type == K44CmdType::ARGMAX_1D) {
                    k44dev::ProgStage f{};
                    f.type = k44dev::PROG_ARGMAX_FINAL;
                    f.items = 1u;
                    f.first = g.first;
                    f.count = 1u;
                    st.push_back(f);
                    st_wr.push_back({});
                }
                continue;
            }
            std::vector<size_t> members;
            if (r.first == 1) members = {r.second};
            else members = groups[r.second]->members;
            g.type = k44dev::PROG_WAVES;
            g.first = (uint32_t)pw.size();
            g.count = (uint32_t)members.size();
            uint32_t items = 0, kq_max = 0;
            Ranges wrs;
            for (size_t m : members) {
                const WaveExec &w = *waves[m];
                if (!w.mfma || !w.narrow || (w.cluster != 64u && w.cluster != 128u) || w.tile2d ||
                    w.mis || w.S % 32u != 0u)
                    return fail("wave '" + w.name + "' is not a narrow wave of 64 / 128-neuron "
                                "tiles over whole 32-position k-steps");
                if (w.out_stride % 4u != 0u || !al(w.y_off_run, 4u) ||
                    (w.has_res && !al(w.res_off, 4u)))
                    return fail("wave '" + w.name + "': output or residual rows are not 8-byte "
                                "aligned");
                if (w.xprod != 0u && w.xprod != 2u && w.xprod != 3u && w.xprod != 4u)
                    return fail("wave '" + w.name + "': gather form " + std::to_string(w.xprod));
                k44dev::ProgWave v{};
                prog_wave_src.push_back(m);
                v.Xo[0] = v.Xo[1] = v.Xo[2] = canvas.p;
                v.seg = w.seg.p;
                v.Wf = w.w.p;
                v.bias = w.bias.p;
                v.cmap = w.cmap.p;
                v.Y = canvas.p + w.y_off_run;
                v.R = w.has_res ? canvas.p + w.res_off : nullptr;
                {
                    const uint32_t nops = w.xprod == 3u ? 3u : w.xprod == 2u ? 2u : 1u;
                    std::vector<Ranges> ops;
                    for (uint32_t k = 0; k < nops; ++k) {
                        const int64_t d = w.xprod ? w.xd[k] : 0;
                        Ranges r;
                        for (const auto &x : w.xrd)
                            r.push_back({(uint64_t)((int64_t)x.first + d),
                                         (uint64_t)((int64_t)x.second + d)});
                        ops.push_back(r);
                    }
                    pw_ops.push_back(ops);
                    pw_res.push_back(w.has_res ? w.resrd : Ranges{});
                    for (const auto &x : w.wr_run) wrs.push_back(x);
                }
                v.step = w.step;
                v.K = w.K;
                v.S = w.S;
                v.ksteps = w.ksteps;
                v.nb = w.cluster / 16u;
                v.tiles = w.rows;
                v.out_stride = w.out_stride;
                v.act = w.act;
                if (w.norm_fold != SIZE_MAX) {
                    const size_t f = w.norm_fold;
                    if (fold_stage[f] != SIZE_MAX && fold_stage[f] != st.size())
                        return fail("the producers of a folded RMSNorm span several launches");
                    fold_stage[f] = st.size();
                }
                wave_fold_in.push_back(w.xnorm);
                if (w.xnorm != SIZE_MAX) {
                    const AuxExec &N = *aux[norm_folds[w.xnorm].norm];
                    v.xgamma = N.table.p;
                    v.xg_base = N.y_off;
                    uint32_t sh = 0;
                    while ((1u << sh) < N.stride) ++sh;
                    v.xg_shift = sh;
                    v.norm_D = N.D;
                    v.norm_eps = N.eps;
                }
                kq_max = std::max(kq_max, (w.ksteps + 3u) / 4u);
                pw.push_back(v);
                g.prod = w.xprod;
            }
            g.kreg = ((kq_max + 7u) / 8u > 1u && (g.prod == 0u || g.prod == 2u)) ? 2u : 1u;
            const uint32_t bpb = k44dev::prog_bpb(g.prod, g.kreg);
            for (uint32_t k = 0; k < g.count; ++k) {
                k44dev::ProgWave &v = pw[g.first + k];
                v.item0 = items;
                items += v.tiles * v.nb / bpb;
            }
            for (size_t m : members) {
                if (waves[m]->xprod != g.prod)
                    return fail("a launch of waves with different gather forms");
                if (waves[m]->norm_fold != waves[members[0]]->norm_fold)
                    return fail("a launch whose waves feed different folded RMSNorms");
            }
            g.items = items;
            st.push_back(g);
            st_wr.push_back(merge_ranges(wrs));
        }
        if (st.empty()) return fail("empty plan");
        uint32_t grid = 0;
        K44_HIP(k44dev::prog_grid(grid));
        uint64_t cum = 0;
        for (auto &g : st) {
            g.rot = (uint32_t)(cum % grid);
            g.base = (uint32_t)cum;
            cum += g.items;
        }
        if (tune(Tune::ProgTrace) == 1) {
            prog_trace.alloc(8u * cum);
            K44_HIP(hipMemsetAsync(prog_trace.p, 0, prog_trace.n * sizeof(uint64_t), stream));
        }
        // Shadow layout: stage t's written span [lo, hi) at shadow element base[t].
        std::vector<uint64_t> sh_lo(st.size(), 0), sh_base(st.size(), 0);
        uint64_t sh_total = 0;
        for (size_t t = 0; t < st.size(); ++t) {
            if (st_wr[t].empty()) continue;
            sh_lo[t] = st_wr[t].front().first;
            sh_base[t] = sh_total;
            sh_total += (st_wr[t].back().second - sh_lo[t] + 63u) / 64u * 64u;
        }
        prog_shadow.alloc(sh_total + 64u);
        // the last stage before `before` that wrote any of `rs`: it must have written all of
        // them (-1: none did, the canvas holds them); -2: no single producer
        auto writer_of = [&](const Ranges &rs, size_t before) -> long {
            long w_all = -3;
            for (const auto &r : rs) {
                long w = -1;
                for (size_t t = before; t-- > 0;)
                    if (ranges_overlap(st_wr[t], Ranges{r})) {
                        w = (long)t;
                        break;
                    }
                if (w >= 0) {
                    bool inside = false;
                    for (const auto &x : st_wr[(size_t)w])
                        inside = inside || (x.first <= r.first && r.second <= x.second);
                    if (!inside) return -2;
                }
                if (w_all == -3) w_all = w;
                else if (w_all != w) return -2;
            }
            return w_all == -3 ? -1 : w_all;
        };
        // element pointer to canvas element offsets of stage w's outputs (shadow or canvas)
        auto base_of = [&](long w) -> __half * {
            if (w < 0) return canvas.p;
            return reinterpret_cast<__half *>(
                reinterpret_cast<uintptr_t>(prog_shadow.p) +
                2u * (uintptr_t)(int64_t)((int64_t)sh_base[(size_t)w] - (int64_t)sh_lo[(size_t)w]));
        };
        for (size_t t = 0; t < st.size(); ++t) {
            const k44dev::ProgStage &g = st[t];
            if (g.type == k44dev::PROG_WAVES) {
                for (uint32_t k = 0; k < g.count; ++k) {
                    const size_t i = g.first + k;
                    k44dev::ProgWave &v = pw[i];
                    const WaveExec &w = *waves[prog_wave_src[i]];
                    for (size_t o = 0; o < pw_ops[i].size(); ++o) {
                        const long wr = writer_of(pw_ops[i][o], t);
                        if (wr == -2) return fail("wave '" + w.name + "' gathers rows of several producers");
                        v.Xo[o] = base_of(wr) + (w.xprod ? w.xd[o] : 0);
                    }
                    if (w.has_res) {
                        const long wr = writer_of(pw_res[i], t);
                        if (wr == -2) return fail("wave '" + w.name + "' adds rows of several producers");
                        v.R = base_of(wr) + w.res_off;
                    }
                    v.Ys = base_of((long)t) + w.y_off_run;
                }
            } else if (g.type != k44dev::PROG_ARGMAX_FINAL) {
                k44dev::ProgAux &x = pa[g.first];
                if (!pa_rd[g.first].empty()) {
                    const long wr = writer_of(pa_rd[g.first], t);
                    if (wr == -2) return fail("a token op reads rows of several producers");
                    x.x = base_of(wr) + pa_rd[g.first].front().first;
                }
                if (x.y) x.ys = base_of((long)t) + (uint64_t)(x.y - canvas.p);
                if (x.y2) x.y2s = base_of((long)t) + (uint64_t)(x.y2 - canvas.p);
            }
        }
        prog_zero.alloc(64u);
        K44_HIP(hipMemsetAsync(prog_zero.p, 0, prog_zero.n * sizeof(uint64_t), stream));
        for (auto &x : pa) x.keys = prog_zero.p;
        // slots of the folded norms: 32 words per item of each producing stage
        std::vector<size_t> slot_off(nfold, 0);
        size_t nslot = 0;
        for (size_t f = 0; f < nfold; ++f) {
            if (fold_stage[f] == SIZE_MAX) continue;
            const k44dev::ProgStage &g = st[fold_stage[f]];
            slot_off[f] = nslot;
            nslot += 32u * (size_t)g.items * k44dev::prog_bpb(g.prod, g.kreg);
        }
        if (nslot) prog_slots.alloc(nslot);
        auto slots_of = [&](size_t f, uint32_t &n) -> uint64_t * {
            if (f == SIZE_MAX || fold_stage[f] == SIZE_MAX) return nullptr;
            const k44dev::ProgStage &g = st[fold_stage[f]];
            n = g.items * k44dev::prog_bpb(g.prod, g.kreg);  // one slot per 16-neuron block
            return prog_slots.p + slot_off[f];
        };
        for (size_t i = 0; i < pa.size(); ++i) {
            uint32_t n = 0;
            pa[i].slot_in = slots_of(aux_fold[i], n);
            pa[i].slot_n = n;
            if (aux_fold[i] != SIZE_MAX && !pa[i].slot_in)
                return fail("a folded RMSNorm whose producers are not in the program");
        }
        {
            size_t i = 0;
            for (const auto &g : st) {
                if (g.type != k44dev::PROG_WAVES) continue;
                for (uint32_t k = 0; k < g.count; ++k, ++i) {
                    k44dev::ProgWave &v = pw[g.first + k];
                    const WaveExec &w = *waves[prog_wave_src[g.first + k]];
                    uint32_t n = 0, dummy = 0;
                    v.slot_out = w.norm_fold != SIZE_MAX ? slots_of(w.norm_fold, dummy) : nullptr;
                    v.slot_in = slots_of(wave_fold_in[g.first + k], n);
                    v.slot_n = n;
                    if (wave_fold_in[g.first + k] != SIZE_MAX && !v.slot_in)
                        return fail("a folded RMSNorm whose producers are not in the program");
                }
            }
        }
        prog_stages_h = st;
        prog_stages.upload(st);
        prog_waves.upload(pw);
        prog_aux.upload(pa);
        prog_ctrs.alloc(st.size() + 2u);
        K44_HIP(hipMemsetAsync(prog_ctrs.p, 0, prog_ctrs.n * sizeof(uint32_t), stream));
        int rate_khz = 0, dev = 0;
        K44_HIP(hipGetDevice(&dev));
        K44_HIP(hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, dev));
        const int spin_ms = tune(Tune::ProgSpinMs) < 0 ? 1000 : tune(Tune::ProgSpinMs);
        prog_args = k44dev::ProgArgs{};
        prog_args.stages = prog_stages.p;
        prog_args.waves = prog_waves.p;
        prog_args.aux = prog_aux.p;
        prog_args.done = prog_ctrs.p;
        prog_args.exit_ctr = prog_ctrs.p + st.size();
        prog_args.abort = prog_ctrs.p + st.size() + 1u;
        prog_args.zero_base = prog_zero.p;
        prog_args.zero_words = (uint32_t)prog_zero.n;
        prog_args.spin_ticks = (uint64_t)std::max(rate_khz, 1) * (uint64_t)spin_ms;
        prog_args.nstages = (uint32_t)st.size();
        prog_args.trace = prog_trace.p;
        K44_HIP(hipStreamSynchronize(stream));
        prog_grid = grid;
        prog_active = true;
        prog_why = "persistent launch: " + std::to_string(st.size()) + " stages, " +
                   std::to_string(grid) + " workgroups";
    }

    // A persistent launch that gave up on a stage wait left a nonzero abort word: report it
    // (and clear it) at the next host synchronisation.
    void check_program() {
        if (!prog_active) return;
        uint32_t ab = 0;
        K44_HIP(hipMemcpyAsync(&ab, prog_args.abort, sizeof(ab), hipMemcpyDeviceToHost, stream));
        K44_HIP(hipStreamSynchronize(stream));
        if (!ab) return;
        K44_HIP(hipMemsetAsync(prog_args.abort, 0, sizeof(uint32_t), stream));
        K44_HIP(hipStreamSynchronize(stream));
        throw std::runtime_error("persistent decode launch abandoned: the wait for stage " +
                                 std::to_string(ab - 1u) + " exceeded its time limit (" +
                                 std::to_string(prog_args.spin_ticks) + " ticks); outputs of "
                                 "that run are incomplete");
    }

    void free_all() {
        // Nothing queued on the executor stream may still use the graph or the buffers.
        if (stream) (void)hipStreamSynchronize(stream);
        drop_graph();
        groups.clear();
        waves.clear();
        aux.clear();
        ops.clear();
        runs.clear();
        wave_cmd.clear();
        aux_cmd.clear();
        ids.reset();
        stage.reset();
        history.reset();
        step_ctr.reset();
        id_tokens = hist_steps = 0;
        canvas.reset();
        scratch.reset();
        scratch_need = 0;
        arrive.reset();
        norm_folds.clear();
        norm_slots.reset();
        norm_ctrs.reset();
        norm_invs.reset();
        fold_elems = 0;
        drop_program("not built");
        if (ev0) (void)hipEventDestroy(ev0);
        if (ev1) (void)hipEventDestroy(ev1);
        if (stream) (void)hipStreamDestroy(stream);
        ev0 = ev1 = nullptr;
        stream = nullptr;
        initialized = false;
    }

    // Index rows -> dendritic segments.  Canvas element offsets e[s] of a row are split at
    // every s where e[s] != e[s-1] + step; the segment length S is the gcd of B_raw and all
    // split points, so every row is K = B_raw / S runs of S consecutive positions.
    // With `reorder`, a row whose synapses in index order give segments shorter than 32
    // positions is also tried in phase order — synapses sorted by (offset mod step, offset) —
    // and that order is kept (perm[r * B_raw + s] = index-order synapse of position s) when it
    // gives longer segments.  A 1-D convolution of kw taps over contiguous channels is such a
    // row: in index order every synapse is its own segment (channel-major, tap-minor offsets
    // ch_base + dx), in phase order it is kw segments of cin consecutive channels.
    static void segment_rows(const K44ExecCmd &c, uint64_t step, uint32_t &S_out,
                             std::vector<uint64_t> &starts, std::vector<uint32_t> &perm,
                             bool reorder) {
        const uint32_t B = c.B, b_raw = c.B_raw;
        const size_t rows = c.h_idx.size() / B;
        std::vector<uint64_t> off((size_t)rows * b_raw);
        for (size_t r = 0; r < rows; ++r)
            for (uint32_t s = 0; s < b_raw; ++s) {
                const uint64_t v = c.h_idx[r * B + s];
                off[r * b_raw + s] = c.idx_mode == 1u ? c.x_base_off + v * c.idx_stride
                                                      : c.x_base_off + v;
            }
        auto seg_len = [&](const std::vector<uint64_t> &o) {
            uint32_t S = b_raw;
            for (size_t r = 0; r < rows && S > 1u; ++r) {
                const uint64_t *e = o.data() + r * b_raw;
                for (uint32_t s = 1; s < b_raw; ++s)
                    if (e[s] != e[s - 1] + step) S = std::gcd(S, s);
            }
            return S;
        };
        uint32_t S = seg_len(off);
        perm.clear();
        if (reorder && S < 32u && b_raw > 1u && step > 1u) {
            std::vector<uint32_t> pm((size_t)rows * b_raw);
            std::vector<uint64_t> po(off.size());
            for (size_t r = 0; r < rows; ++r) {
                uint32_t *q = pm.data() + r * b_raw;
                const uint64_t *e = off.data() + r * b_raw;
                for (uint32_t s = 0; s < b_raw; ++s) q[s] = s;
                std::stable_sort(q, q + b_raw, [&](uint32_t x, uint32_t y) {
                    const uint64_t px = e[x] % step, py = e[y] % step;
                    return px != py ? px < py : e[x] < e[y];
                });
                for (uint32_t s = 0; s < b_raw; ++s) po[r * b_raw + s] = e[q[s]];
            }
            const uint32_t Sp = seg_len(po);
            if (Sp > S) {
                S = Sp;
                off.swap(po);
                perm.swap(pm);
            }
        }
        const uint32_t K = b_raw / S;
        starts.resize(rows * K);
        for (size_t r = 0; r < rows; ++r)
            for (uint32_t k = 0; k < K; ++k) starts[r * K + k] = off[r * b_raw + (size_t)k * S];
        S_out = S;
    }

    // VALU gathers whose distinct rows are far beyond the caches (>= 512 MiB, twice the MALL)
    // read their rows and weights with the non-temporal load policy: config 2 (random 8 KiB
    // segments of a 20 GB substrate) 391 -> 373 us.  Cache-resident substrates keep the default
    // policy.  Tuning switch "nt" forces either.
    static bool streaming_gather(const WaveExec &wx) {
        if (tune(Tune::NonTemporal) >= 0) return tune(Tune::NonTemporal) == 1;
        return wx.unique_rows * (uint64_t)wx.tokens * 2u >= (512ull << 20);
    }

    // MFMA configuration of a wave with a dense tiling (tiles of cl = cluster_size neurons
    // sharing every index row): kernel (narrow <= 16 tokens, LDS ring for 512-token
    // workgroups, register-staged tile otherwise), ring depth, split-K, and the weights in
    // A-fragment order.  width: the output's token count per row (1-D waves; 2-D waves pass
    // UINT32_MAX: they never take the narrow kernel).
    void configure_mfma(const K44ExecCmd &c, WaveExec &wx, const std::vector<uint16_t> &wraw,
                        size_t rows, uint32_t width) {
        const uint32_t cl = c.cluster_size;
        wx.path = "mfma_tile";
        wx.why = "neurons share index rows in tiles of " + std::to_string(cl) +
                 " and segments are whole 32-position K-steps: dense " + std::to_string(cl) +
                 " x " + std::to_string(c.B_raw) + " x " + std::to_string(wx.tokens) +
                 " contraction per tile on v_mfma_f32_16x16x32_f16";
        wx.mt = pick_mt(wx.tokens);
        wx.rows_per_stage = (wx.S % 64u == 0u && cl <= 64u && !wx.mis) ? 64u : 32u;
        // Rows off the 16-byte grid take the register-staged tile kernel (its loads pass
        // through registers, where they are shifted into place); the narrow and LDS-ring
        // kernels gather aligned rows only.
        wx.narrow = width <= 16u && tune(Tune::Narrow) != 0 && !wx.mis;
        wx.part_tokens = wx.narrow ? 16u : wx.tokens;
        // 512-token workgroups of 32/64-neuron tiles stream through an LDS ring filled by
        // direct loads (3 stages in flight per workgroup instead of 1).
        wx.dma = !wx.narrow && !wx.mis && wx.mt == 512u &&
                 (cl == 32u || cl == 64u || cl == 128u) && tune(Tune::Dma) != 0;
        if (wx.mis)
            wx.why += " (rows off the 16-byte grid: aligned loads shifted into place, 32-row "
                      "stages)";
        if (wx.dma) {
            wx.path = "mfma_dma";
            wx.why += " (512-token workgroups: 4-stage LDS ring filled by global_load_lds)";
            wx.rows_per_stage = 32u;
            // Config 3 measured the same with either load policy (363 TFLOP/s): default
            // policy unless tuning switch "nt" is 1.
            wx.stream_loads = tune(Tune::NonTemporal) == 1;
            // Ring depth: gathers from inputs that stay in the caches (distinct gathered
            // bytes <= 256 MB, the last-level cache) take 2-stage rings, two workgroups per
            // CU — config-5 prefill 26.9 -> 20.9 ms; gathers from HBM keep 4 stages and one
            // workgroup per CU — config 3: 364 us, against 379 us with 2 stages.
            const double gathered = (double)wx.unique_rows * wx.tokens * 2.0;
            wx.dshape.nbuf = gathered <= 256.0 * 1048576.0 ? 2u : 4u;
            if (tune(Tune::DmaStages) == 2 || tune(Tune::DmaStages) == 4)
                wx.dshape.nbuf = (uint32_t)tune(Tune::DmaStages);
            // 128-neuron tiles: 128 accumulator registers per lane leave one workgroup per
            // CU, whose LDS holds a 3-stage ring (2 stages in flight).
            if (cl == 128u) wx.dshape.nbuf = 3u;
            // Producer waves issue every load of a stage, the 8 other waves only multiply:
            // a 4-stage ring, one workgroup of 8 + P waves per CU (32/64-neuron tiles).
            if (tune(Tune::DmaProd) == 1 && cl != 128u) {
                wx.dshape.prod = cl == 32u ? 2u : 4u;
                wx.dshape.nbuf = 4u;
            }
            wx.dshape.stream_loads = wx.stream_loads;
            wx.why += "; " + std::to_string(wx.dshape.nbuf) + "-stage ring";
            if (wx.dshape.prod)
                wx.why += ", " + std::to_string(wx.dshape.prod) + " producer waves";
        }
        if (wx.narrow) {
            wx.path = "mfma_narrow";
            wx.why += " (at most 16 tokens: weight-streaming narrow tile)";
            wx.mt = 16u;
            const uint32_t ksteps = c.B_raw / 32u;
            uint32_t want;
            if (cl >= 64u) {
                // Tiles of whole 16-neuron blocks per wave: chunks of any length, streamed
                // in 16-k-step sub-chunks.  Chunks of at most 48 k-steps; split further, down
                // to 16 k-steps, until the wave has ~64 workgroups (~128 when a second kernel
                // reduces the partials).  Measured on config-5 decode (ms per step, graph
                // replays, alternated in one process): partials reduced by the tile's last
                // workgroup 0.869 at 64 workgroups, 0.889 at 32, 0.941 at 128, 0.968 unsplit
                // beyond 48 k-steps; reduced by the epilogue kernel 0.928 at 128 or 64.
                const int ce = tune(Tune::NarrowChunk), cw = tune(Tune::NarrowWgs);
                const uint32_t cmax = ce > 0 ? (uint32_t)std::max(16, ce) : 48u;
                const uint32_t wgs =
                    cw > 0 ? (uint32_t)cw : (tune(Tune::NarrowReduce) != 0 ? 64u : 128u);
                want = (ksteps + cmax - 1u) / cmax;
                want = std::max(want, std::min((wgs + (uint32_t)rows - 1u) / (uint32_t)rows,
                                               (ksteps + 15u) / 16u));
            } else {
                // Chunks of 8..16 k-steps (<= 512 rows in LDS), ~256 workgroups per wave.
                want = (256u + (uint32_t)rows - 1u) / (uint32_t)rows;
                want = std::min(want, (ksteps + 7u) / 8u);
                want = std::max(want, (ksteps + 15u) / 16u);
            }
            want = std::max(1u, std::min(want, ksteps));
            wx.stage_chunk = (ksteps + want - 1u) / want;
            wx.kgroups = (ksteps + wx.stage_chunk - 1u) / wx.stage_chunk;
            if (wx.kgroups > 1u) wx.part_floats = (size_t)wx.kgroups * c.Cout * 16u;
            // Split 64/128-neuron tiles: the tile's last workgroup reduces (no epilogue kernel).
            wx.reduce_in_kernel = cl >= 64u && wx.kgroups > 1u && tune(Tune::NarrowReduce) != 0;
        } else {
            const uint32_t stages = c.B_raw / wx.rows_per_stage;
            const uint64_t wgs = (uint64_t)rows * (wx.tokens / wx.mt);
            // Few workgroups: split the contraction.  Each split adds a partial plane of
            // 4 * cout * tokens bytes, so prefill-sized token counts split at most 8 ways
            // with >= 4 stages per workgroup; small token counts up to 32 ways.
            const bool wide_tokens = wx.tokens >= 1024u;
            uint32_t want = wgs >= 256u ? 1u : (uint32_t)((512u + wgs - 1u) / wgs);
            if (tune(Tune::SplitK) == 0) want = 1u;
            want = std::min(want, wide_tokens ? 8u : 32u);
            const uint32_t min_stages = wide_tokens ? 4u : 1u;
            want = std::max(1u, std::min(want, std::max(1u, stages / min_stages)));
            wx.stage_chunk = (stages + want - 1u) / want;
            wx.kgroups = (stages + wx.stage_chunk - 1u) / wx.stage_chunk;
            if (wx.kgroups > 1u) wx.part_floats = (size_t)wx.kgroups * c.Cout * wx.tokens;
        }
        wx.ksteps = c.B_raw / 32u;
        const uint32_t nb = cl / 16u;
        // A fragments: [tile][k-step][16-neuron block][lane][8]; lane l holds neuron
        // 16*blk + (l & 15), positions 32*ks + 8*(l >> 4) .. +8 of the tile's index row.
        std::vector<uint16_t> wf((size_t)c.Cout * c.B_raw);
        for (size_t t = 0; t < rows; ++t)
            for (uint32_t ks = 0; ks < wx.ksteps; ++ks)
                for (uint32_t b = 0; b < nb; ++b)
                    for (uint32_t l = 0; l < 64u; ++l) {
                        const size_t dst = (((t * wx.ksteps + ks) * nb + b) * 64u + l) * 8u;
                        const size_t j = t * cl + 16u * b + (l & 15u);
                        const size_t src = j * c.B + 32u * ks + 8u * (l >> 4);
                        std::memcpy(&wf[dst], &wraw[src], 16);
                    }
        std::vector<__half> wh(wf.size());
        std::memcpy(wh.data(), wf.data(), wf.size() * 2u);
        wx.w.upload(wh);
    }

    void build_wave(const K44ExecCmd &c, WaveExec &wx) {
        const auto &Lo = plan_meta.res_map.at(c.res_key_out);
        auto itin = plan_meta.res_map.find(c.res_key_in);
        if (itin == plan_meta.res_map.end())
            throw std::runtime_error("wave '" + c.name + "': unknown input layout");
        if (!Lo.is_1d_tokens || !itin->second.is_1d_tokens) {
            build_wave2d(c, wx, Lo, itin->second);
            return;
        }
        if (c.h_idx.empty() || c.B == 0u || c.B_raw == 0u || c.h_idx.size() % c.B != 0u)
            throw std::runtime_error("wave '" + c.name + "': missing or malformed index table");
        if (c.h_w_wmma.size() * 8u < (size_t)c.Cout * c.B)
            throw std::runtime_error("wave '" + c.name + "': weight block smaller than Cout x B");
        const size_t rows = c.h_idx.size() / c.B;
        if (rows * c.cluster_size != c.Cout)
            throw std::runtime_error("wave '" + c.name + "': index rows x cluster != Cout");
        if (c.has_cout_map && c.h_cout_map.size() < c.Cout)
            throw std::runtime_error("wave '" + c.name + "': cout_map shorter than Cout");

        wx.name = c.name;
        wx.cout = c.Cout;
        wx.cluster = c.cluster_size;
        wx.rows = (uint32_t)rows;
        wx.tokens = Lo.channel_stride;  // single-frame 1-D: tiles 64t .. 64t+63 of the row
        wx.out_stride = Lo.channel_stride;
        wx.step = c.idx_mode == 1u ? c.idx_stride : itin->second.channel_stride;
        wx.y_off = c.y_off;
        wx.res_off = c.res_off;
        wx.has_res = c.has_residual;
        wx.act = (int)c.act;
        if (wx.act < 0 || wx.act > 5)
            throw std::runtime_error("wave '" + c.name + "': unknown activation id");

        std::vector<uint64_t> starts;
        std::vector<uint32_t> perm;
        segment_rows(c, wx.step, wx.S, starts, perm, true);
        wx.K = c.B_raw / wx.S;
        wx.phase_order = !perm.empty();

        // Row-major [Cout][B] weights from the on-disk WMMA order; padded synapses must be 0.
        std::vector<uint16_t> wraw((size_t)c.Cout * c.B);
        convert_wmma_to_raw(reinterpret_cast<uint4_host *>(wraw.data()), c.h_w_wmma.data(),
                            c.Cout, c.B / 8u);
        for (size_t j = 0; j < c.Cout; ++j)
            for (uint32_t s = c.B_raw; s < c.B; ++s)
                if (wraw[j * c.B + s] != 0u)
                    throw std::runtime_error("wave '" + c.name +
                                             "': non-zero weight on a padded synapse");
        if (!perm.empty()) {  // synapses in the segment order chosen above
            std::vector<uint16_t> tmp(c.B_raw);
            for (size_t j = 0; j < c.Cout; ++j) {
                const uint32_t *q = perm.data() + (j / c.cluster_size) * c.B_raw;
                uint16_t *wj = wraw.data() + j * c.B;
                for (uint32_t s = 0; s < c.B_raw; ++s) tmp[s] = wj[q[s]];
                std::memcpy(wj, tmp.data(), (size_t)c.B_raw * 2u);
            }
        }

        // Address-sorted segments: every index row visits its segments in ascending canvas
        // order (weight columns permuted with them; only the fp32 summation order changes), so
        // concurrently running rows sweep the substrate together and overlapping segments of
        // different rows are read close in time (cache reuse instead of a second HBM read).
        wx.sorted_segments = wx.K > 1u && tune(Tune::SortSegments) != 0;
        if (wx.sorted_segments) {
            std::vector<uint32_t> order(wx.K);
            std::vector<uint64_t> st(wx.K);
            std::vector<uint16_t> row_w((size_t)c.B_raw);
            for (size_t r = 0; r < rows; ++r) {
                uint64_t *sr = starts.data() + r * wx.K;
                for (uint32_t k = 0; k < wx.K; ++k) order[k] = k;
                std::stable_sort(order.begin(), order.end(),
                                 [&](uint32_t x, uint32_t y) { return sr[x] < sr[y]; });
                bool identity = true;
                for (uint32_t k = 0; k < wx.K; ++k) identity = identity && order[k] == k;
                if (identity) continue;
                for (uint32_t k = 0; k < wx.K; ++k) st[k] = sr[order[k]];
                std::copy(st.begin(), st.end(), sr);
                for (size_t j = r * c.cluster_size; j < (r + 1) * c.cluster_size; ++j) {
                    uint16_t *wj = wraw.data() + j * c.B;
                    for (uint32_t k = 0; k < wx.K; ++k)
                        std::memcpy(&row_w[(size_t)k * wx.S], wj + (size_t)order[k] * wx.S,
                                    wx.S * 2u);
                    std::memcpy(wj, row_w.data(), (size_t)c.B_raw * 2u);
                }
            }
        }

        // Token-shifted taps: segment starts off the 4-element (8-byte) grid take the funnel-
        // shift gather, whose second word reads up to 3 elements past a row's last token.
        for (uint64_t s0 : starts) wx.misaligned = wx.misaligned || s0 % 4u != 0u;
        // Host-side bounds check of every canvas element the kernel may touch.
        const uint64_t n_canvas = plan_meta.canvas_elems;
        uint64_t x_hi = 0;
        for (uint64_t s0 : starts) x_hi = std::max(x_hi, s0);
        x_hi += (uint64_t)(wx.S - 1u) * wx.step + wx.tokens;
        // Rows off the 16-byte grid are read as the aligned 16-byte chunks around them: up to 16
        // elements past a row's last token, inside the canvas's slack.
        bool off16 = false;
        for (uint64_t s0 : starts) off16 = off16 || s0 % 8u != 0u;
        if (x_hi + (off16 ? 16u : 0u) > n_canvas + (off16 ? kCanvasSlack : 0u))
            throw std::runtime_error("wave '" + c.name + "': gather reaches past the canvas");
        uint64_t oj_hi = c.Cout - 1u;
        if (c.has_cout_map) {
            oj_hi = 0;
            for (uint32_t j = 0; j < c.Cout; ++j)
                if (c.h_cout_map[j] != 0xffffu)  // empty slot: the kernels store nothing
                    oj_hi = std::max<uint64_t>(oj_hi, c.h_cout_map[j]);
        }
        const uint64_t span = oj_hi * wx.out_stride + wx.tokens;
        if (wx.y_off + span > n_canvas || (wx.has_res && wx.res_off + span > n_canvas))
            throw std::runtime_error("wave '" + c.name + "': output/residual past the canvas");
        if (wx.tokens % 64u != 0u || wx.out_stride % 4u != 0u || wx.y_off % 4u != 0u ||
            wx.res_off % 4u != 0u || wx.step % 4u != 0u)
            throw std::runtime_error("wave '" + c.name + "': canvas rows not 8-byte aligned");

        {
            Ranges rd, wr;
            rd.reserve(starts.size() + c.Cout);
            const uint64_t over = wx.misaligned ? 4u : 0u;  // funnel-shift words past the row
            for (uint64_t s0 : starts)
                rd.push_back({s0, s0 + (uint64_t)(wx.S - 1u) * wx.step + wx.tokens + over});
            for (uint32_t j = 0; j < c.Cout; ++j) {
                const uint64_t oj = c.has_cout_map ? (uint64_t)c.h_cout_map[j] : (uint64_t)j;
                if (c.has_cout_map && oj == 0xffffu) continue;
                wr.push_back({wx.y_off + oj * wx.out_stride, wx.y_off + oj * wx.out_stride + wx.tokens});
                if (wx.has_res)
                    rd.push_back({wx.res_off + oj * wx.out_stride,
                                  wx.res_off + oj * wx.out_stride + wx.tokens});
            }
            Ranges xr;
            xr.reserve(starts.size());
            for (uint64_t s0 : starts)
                xr.push_back({s0, s0 + (uint64_t)(wx.S - 1u) * wx.step + wx.tokens});
            wx.xrd = merge_ranges(std::move(xr));
            Ranges rr;
            if (wx.has_res)
                for (uint32_t j = 0; j < c.Cout; ++j) {
                    const uint64_t oj = c.has_cout_map ? (uint64_t)c.h_cout_map[j] : (uint64_t)j;
                    if (c.has_cout_map && oj == 0xffffu) continue;
                    rr.push_back({wx.res_off + oj * wx.out_stride,
                                  wx.res_off + oj * wx.out_stride + wx.tokens});
                }
            wx.resrd = merge_ranges(std::move(rr));
            wx.rd = merge_ranges(std::move(rd));
            wx.wr = merge_ranges(std::move(wr));
            wx.rd_run = wx.rd;
            wx.wr_run = wx.wr;
            wx.y_off_run = wx.y_off;
        }

        // Distinct substrate positions (compulsory-traffic accounting).
        {
            std::vector<std::pair<uint64_t, uint64_t>> iv;
            iv.reserve(starts.size());
            for (uint64_t s0 : starts) iv.push_back({s0, s0 + (uint64_t)wx.S * wx.step});
            std::sort(iv.begin(), iv.end());
            uint64_t covered = 0, cur_lo = 0, cur_hi = 0;
            bool open = false;
            for (auto &p : iv) {
                if (!open || p.first > cur_hi) {
                    if (open) covered += cur_hi - cur_lo;
                    cur_lo = p.first;
                    cur_hi = p.second;
                    open = true;
                } else {
                    cur_hi = std::max(cur_hi, p.second);
                }
            }
            if (open) covered += cur_hi - cur_lo;
            wx.unique_rows = wx.step ? covered / wx.step : 0;
        }

        // Path selection.  MFMA needs a real dense contraction: >= 16 neurons sharing every
        // index row (tile NT in {16, 32, 64, 128}), segments of whole 32-deep K-steps and
        // 16-byte aligned rows.  Everything else is a batched GEMV: VALU gather-dot.
        const int force = tune(Tune::Path);  // -1 auto, 0 VALU, 1 MFMA
        bool aligned8 = wx.step % 8u == 0u;
        for (uint64_t s0 : starts) aligned8 = aligned8 && s0 % 8u == 0u;
        const uint32_t cl = c.cluster_size;
        const bool nt_ok = cl == 16u || cl == 32u || cl == 64u || cl == 128u;
        // Segment starts off the 16-byte grid (token-shifted taps): the MIS tile kernel, as long
        // as consecutive positions of a segment stay 16 bytes apart (step % 8 == 0).
        const bool mfma_ok =
            nt_ok && wx.S % 32u == 0u && wx.step % 8u == 0u && wx.tokens % 64u == 0u;
        wx.mfma = mfma_ok && force != 0;
        wx.mis = wx.mfma && !aligned8;
        if (force == 1 && !mfma_ok)
            throw std::runtime_error("wave '" + c.name + "': tuning path=mfma but the wave has "
                                     "no dense MFMA tiling (cluster/segment/alignment)");
        if (wx.mfma) {
            configure_mfma(c, wx, wraw, rows, Lo.W);
        } else {
            wx.path = "valu_gather_dot";
            wx.why = !nt_ok ? "neurons do not share index rows in tiles of 16..128 (cluster " +
                                  std::to_string(cl) + "): no dense contraction, batched GEMV"
                     : wx.S % 32u != 0u
                         ? "segments of " + std::to_string(wx.S) +
                               " positions do not fill 32-deep MFMA K-steps"
                         : (force == 0 ? std::string("forced by tuning switch path=0")
                                  : std::string("positions of a segment not 16 bytes apart"));
            if (wx.misaligned)
                wx.why += "; token-shifted segment starts: funnel-shift gathers, 4 tokens per lane";
            if (wx.phase_order) wx.why += "; synapses regrouped by token phase";
            wx.slab = pick_slab(wx.tokens);
            {
                // 8 tokens per lane (16-byte loads) when the rows it gathers fit the 256 MB MALL
                // (measured: configs 1 and 4 13-28 % faster); 4 tokens per lane for HBM-bound
                // gathers (config 2: 2.5 % faster).  16-byte accesses need 8-element alignment.
                const bool want8 = tune(Tune::Lane8) >= 0
                                       ? tune(Tune::Lane8) == 1
                                       : wx.unique_rows * (uint64_t)wx.tokens * 2u < (256ull << 20);
                bool ok8 = wx.out_stride % 8u == 0u && wx.y_off % 8u == 0u &&
                           wx.res_off % 8u == 0u && wx.step % 8u == 0u && !wx.misaligned;
                for (uint64_t s0 : starts) ok8 = ok8 && s0 % 8u == 0u;
                wx.lane8 = want8 && ok8;
                wx.stream_loads = streaming_gather(wx);
                wx.weights_in_lds = tune(Tune::WeightsInLds) != 0;
            }
            // Four waves per neuron (segments round-robin) for few-segment neurons gathering from
            // HBM; one wave per neuron when the rows are cache resident (8 tokens per lane,
            // weights in LDS): config 1 19.2 us against 23.2 us with four.
            wx.ksplit = (!wx.lane8 && wx.K >= 2u && wx.K <= 8u) ? 4u : 1u;
            if (tune(Tune::KSplit) >= 0) wx.ksplit = tune(Tune::KSplit) == 4 ? 4u : 1u;
            {
                // Streaming gathers over 256-token slabs with >= 256 workgroups of 256 neurons:
                // stage the output rows in LDS and write them after the last gather (writes
                // interleaved with the random reads cost ~15 % on config 2).
                const bool big = (uint64_t)(c.Cout / 256u) * (wx.tokens / 256u) >= 256u;
                const int sk = tune(Tune::StreamKernel);
                wx.stream_kernel = wx.stream_loads && !wx.lane8 && wx.slab == 256u &&
                                   !wx.has_res && !wx.misaligned && (sk >= 0 ? sk == 1 : big);
                if (wx.stream_kernel) {
                    wx.ksplit = 1u;
                    wx.why += "; streaming kernel: 256 neurons per workgroup, output rows "
                              "staged in LDS";
                }
            }
            const uint32_t rpi = 256u / wx.slab;
            wx.U = 16u / rpi;
            const uint32_t per_batch = rpi * wx.U;
            wx.n_batch = (wx.S + per_batch - 1u) / per_batch;
            std::vector<uint16_t> wk((size_t)c.Cout * wx.K * wx.n_batch * per_batch, 0u);
            for (size_t j = 0; j < c.Cout; ++j)
                for (uint32_t k = 0; k < wx.K; ++k)
                    for (uint32_t s = 0; s < wx.S; ++s) {
                        const uint32_t b = s / per_batch, q = s % per_batch;  // q = g*U + u
                        wk[((j * wx.K + k) * wx.n_batch + b) * per_batch + q] =
                            wraw[j * c.B + (size_t)k * wx.S + s];
                    }
            std::vector<__half> wh(wk.size());
            std::memcpy(wh.data(), wk.data(), wk.size() * 2u);
            wx.w.upload(wh);
        }
        wx.seg.upload(starts);
        std::vector<__half> bh(c.Cout);
        for (size_t j = 0; j < c.Cout; ++j) {
            const uint16_t v = j < c.h_bias.size() ? c.h_bias[j] : 0u;
            std::memcpy(&bh[j], &v, 2);
        }
        if (c.has_bias) wx.bias.upload(bh);
        if (c.has_cout_map)
            wx.cmap.upload(std::vector<uint16_t>(c.h_cout_map.begin(), c.h_cout_map.begin() + c.Cout));
        wx.flops = 2.0 * (double)c.Cout * c.B_raw * wx.tokens;
        wx.eff_flops = c.gflops * 1e9;
    }

    // 2-D wave: every 64-token tile of the output layout gathers X at
    // seg + s*step + tile_x[t] + m (tap-shifted, any alignment) and stores pixels at
    // y_off + out_j*channel_stride + tile_y[t] + m.
    void build_wave2d(const K44ExecCmd &c, WaveExec &wx, const K44ResDesc &Lo,
                      const K44ResDesc &Li) {
        const bool tok64 = Lo.is_image_token64;
        if (Li.is_image_token64 != tok64 || Lo.is_1d_tokens || Li.is_1d_tokens)
            throw std::runtime_error("wave '" + c.name + "': mixed 2-D layouts");
        // Input layout: the output's, except for the 64-frame interleaved layout's stride-2
        // convolutions, which gather the input directly (every output pixel reads the input
        // pixels around twice its coordinates).
        const bool stride2 = tok64 && c.res_key_in != c.res_key_out;
        if (!tok64 && c.res_key_in != c.res_key_out)
            throw std::runtime_error("wave '" + c.name +
                                     "': 2-D wave whose input and output layouts differ");
        if (stride2 && (Lo.H != (Li.H + 1u) / 2u || Lo.W != (Li.W + 1u) / 2u))
            throw std::runtime_error("wave '" + c.name + "': stride-2 output size");
        if (tok64 && (Lo.batch_size % 64u != 0u || Li.batch_size != Lo.batch_size))
            throw std::runtime_error("wave '" + c.name + "': interleaved frames not whole blocks");
        if (c.h_idx.empty() || c.B == 0u || c.B_raw == 0u || c.h_idx.size() % c.B != 0u)
            throw std::runtime_error("wave '" + c.name + "': missing or malformed index table");
        if (c.h_w_wmma.size() * 8u < (size_t)c.Cout * c.B)
            throw std::runtime_error("wave '" + c.name + "': weight block smaller than Cout x B");
        const size_t rows = c.h_idx.size() / c.B;
        if (rows * c.cluster_size != c.Cout)
            throw std::runtime_error("wave '" + c.name + "': index rows x cluster != Cout");
        if (c.has_cout_map && c.h_cout_map.size() < c.Cout)
            throw std::runtime_error("wave '" + c.name + "': cout_map shorter than Cout");
        if (!tok64 &&
            (Lo.h_tile_off_X.size() != Lo.num_tiles || Lo.h_tile_off_Y.size() != Lo.num_tiles))
            throw std::runtime_error("wave '" + c.name + "': tile tables missing");
        wx.tile2d = true;
        wx.name = c.name;
        wx.path = "valu_gather_tile";
        wx.why = tok64 ? "2-D layout of 64-frame interleaved images: one 64-token tile per pixel "
                         "(its 64 frames), taps shift whole pixels"
                       : "2-D spatial layout: tap-shifted gathers over padded-plane tiles";
        wx.cout = c.Cout;
        wx.cluster = c.cluster_size;
        wx.rows = (uint32_t)rows;
        wx.step = Li.channel_stride;
        wx.y_off = c.y_off;
        wx.res_off = c.res_off;
        wx.has_res = c.has_residual;
        wx.act = (int)c.act;
        if (wx.act < 0 || wx.act > 5)
            throw std::runtime_error("wave '" + c.name + "': unknown activation id");
        std::vector<uint64_t> starts;
        std::vector<uint32_t> perm;  // phase order: a kh x kw conv is kh*kw segments of cin rows
        segment_rows(c, wx.step, wx.S, starts, perm, true);
        wx.K = c.B_raw / wx.S;
        wx.phase_order = !perm.empty();
        wx.plane = plane_of(Lo);
        std::vector<uint32_t> tx, ty;
        if (tok64) {
            // Tile = (64-frame block, output pixel): the pixel's 64 frames at
            // ((y+1)*W_pad + x+1)*64 of the block; the gather anchor is the input pixel
            // diagonally before the tap centre, (y-1, x-1) (stride 1) or (2y-1, 2x-1) (stride 2),
            // to which the index words add ((1+dy)*W_pad + (1+dx))*64.
            const uint32_t blocks = Lo.batch_size / 64u, f = stride2 ? 2u : 1u;
            wx.masked = 0;
            wx.tiles_per_frame = Lo.H * Lo.W;
            wx.tiles = blocks * wx.tiles_per_frame;
            const uint64_t hi = (uint64_t)blocks * 64u * std::max(Li.single_stride, Lo.single_stride);
            if (hi > 0xffffffffull)
                throw std::runtime_error("wave '" + c.name + "': interleaved plane beyond 32 bits");
            tx.resize(wx.tiles);
            ty.resize(wx.tiles);
            for (uint32_t b = 0; b < blocks; ++b)
                for (uint32_t y = 0; y < Lo.H; ++y)
                    for (uint32_t x = 0; x < Lo.W; ++x) {
                        const size_t t = ((size_t)b * Lo.H + y) * Lo.W + x;
                        tx[t] = (uint32_t)(b * 64ull * Li.single_stride +
                                           ((uint64_t)f * y * Li.W_pad + (uint64_t)f * x) * 64u);
                        ty[t] = (uint32_t)(b * 64ull * Lo.single_stride +
                                           ((uint64_t)(y + 1u) * Lo.W_pad + x + 1u) * 64u);
                    }
        } else {
            wx.masked = Lo.needs_mask ? 1 : 0;
            wx.tiles = Lo.num_tiles;
            wx.tiles_per_frame = Lo.tiles_per_frame;
            tx.resize(Lo.num_tiles);
            ty.resize(Lo.num_tiles);
            for (uint32_t t = 0; t < Lo.num_tiles; ++t) {
                tx[t] = Lo.h_tile_off_X[t];
                const uint32_t fr = t / Lo.tiles_per_frame, tl = t % Lo.tiles_per_frame;
                ty[t] = Lo.needs_mask ? fr * Lo.single_stride + Lo.W_pad + 4u + 64u * tl
                                      : Lo.h_tile_off_Y[t];
            }
        }
        wx.tokens = wx.tiles * 64u;
        wx.out_stride = (uint32_t)Lo.channel_stride;
        // Host-side bounds check of every element the kernel may touch.
        const uint64_t n_canvas = plan_meta.canvas_elems;
        const uint64_t tx_hi = *std::max_element(tx.begin(), tx.end());
        const uint64_t ty_hi = *std::max_element(ty.begin(), ty.end());
        uint64_t x_hi = 0;
        for (uint64_t s0 : starts) x_hi = std::max(x_hi, s0);
        x_hi += (uint64_t)(wx.S - 1u) * wx.step + tx_hi + 64u + 16u;  // + the shifted chunks
        if (x_hi > n_canvas + kCanvasSlack)
            throw std::runtime_error("wave '" + c.name + "': gather reaches past the canvas");
        uint64_t oj_hi = c.Cout - 1u;
        if (c.has_cout_map) {
            oj_hi = 0;
            for (uint32_t j = 0; j < c.Cout; ++j)
                if (c.h_cout_map[j] != 0xffffu) oj_hi = std::max<uint64_t>(oj_hi, c.h_cout_map[j]);
        }
        const uint64_t span = oj_hi * Lo.channel_stride + ty_hi + 64u;
        if (wx.y_off + span > n_canvas || (wx.has_res && wx.res_off + span > n_canvas) ||
            wx.y_off + (uint64_t)c.Cout * Lo.channel_stride > n_canvas)
            throw std::runtime_error("wave '" + c.name + "': output/residual past the canvas");
        // Weights in synapse order (the gather walks synapses p = k*S + s of the row).
        std::vector<uint16_t> wraw((size_t)c.Cout * c.B);
        convert_wmma_to_raw(reinterpret_cast<uint4_host *>(wraw.data()), c.h_w_wmma.data(),
                            c.Cout, c.B / 8u);
        std::vector<__half> wh((size_t)c.Cout * c.B_raw);
        std::vector<uint16_t> tmp(c.B_raw);
        for (size_t j = 0; j < c.Cout; ++j) {
            for (uint32_t q = c.B_raw; q < c.B; ++q)
                if (wraw[j * c.B + q] != 0u)
                    throw std::runtime_error("wave '" + c.name +
                                             "': non-zero weight on a padded synapse");
            uint16_t *wj = wraw.data() + j * c.B;
            if (!perm.empty()) {  // synapses in the segment order chosen above
                const uint32_t *q = perm.data() + (j / c.cluster_size) * c.B_raw;
                for (uint32_t s = 0; s < c.B_raw; ++s) tmp[s] = wj[q[s]];
                std::memcpy(wj, tmp.data(), (size_t)c.B_raw * 2u);
            }
            std::memcpy(&wh[j * c.B_raw], wj, (size_t)c.B_raw * 2u);
        }
        // Dense convolutions (tiles of >= 16 output channels sharing every index row, whole
        // 32-channel k-steps) run on MFMA through the tile tables.  64-frame interleaved
        // images: every tile is a pixel's 64 frames, 64-element aligned.  Single-frame planes:
        // tiles and tap shifts sit at any element offset (rows shifted into place, the MIS
        // tile kernel), halo columns of masked tiles are not stored (MfmaTileArgs::mask_w),
        // and the stores are 2-byte (tile offsets off the 8-byte grid), so these waves run
        // unsplit (the split-K epilogue stores 4 tokens at a time).
        {
            const uint32_t cl = c.cluster_size;
            const bool ok = (cl == 16u || cl == 32u || cl == 64u || cl == 128u) &&
                            wx.S % 32u == 0u && wx.step % 8u == 0u && tune(Tune::Path) != 0;
            bool al = tok64;
            for (uint64_t s0 : starts) al = al && s0 % 8u == 0u;
            for (uint32_t v : tx) al = al && v % 64u == 0u;
            for (uint32_t v : ty) al = al && v % 64u == 0u;
            if (ok && (al || !tok64)) {
                wx.mfma = true;
                wx.mis = !al;
                wx.epi_scalar = !tok64;
                configure_mfma(c, wx, wraw, rows, UINT32_MAX);
                if (wx.epi_scalar) set_split(wx, 1u);
                wx.why += tok64 ? std::string("; 64-frame interleaved image: tile tables")
                                : std::string("; single-frame image: tile tables, rows shifted "
                                              "into place") +
                                      (wx.masked ? ", halo columns not stored" : "");
            }
        }
        if (!wx.mfma) wx.w.upload(wh);
        wx.seg.upload(starts);
        std::vector<__half> bh(c.Cout);
        for (size_t j = 0; j < c.Cout; ++j) {
            const uint16_t v = j < c.h_bias.size() ? c.h_bias[j] : 0u;
            std::memcpy(&bh[j], &v, 2);
        }
        if (c.has_bias) wx.bias.upload(bh);
        if (c.has_cout_map)
            wx.cmap.upload(std::vector<uint16_t>(c.h_cout_map.begin(), c.h_cout_map.begin() + c.Cout));
        wx.tile_x.upload(tx);
        wx.tile_y.upload(ty);
        wx.flops = 2.0 * (double)c.Cout * c.B_raw * Lo.H * Lo.W * Lo.batch_size;
        wx.eff_flops = c.gflops * 1e9;
    }

    // 2-D spatial aux commands (reference k44_wave_executor.cu:480-544).
    void build_spatial(const K44ExecCmd &c, AuxExec &ax) {
        const K44ResDesc &Li = plan_meta.res_map.at(c.res_key_in);
        const K44ResDesc &Lo = plan_meta.res_map.at(c.res_key_out);
        if (Li.is_1d_tokens || Lo.is_1d_tokens || Li.is_image_token64 != Lo.is_image_token64)
            throw std::runtime_error("command '" + c.name + "': needs matching 2-D layouts");
        if (Li.batch_size != Lo.batch_size)
            throw std::runtime_error("command '" + c.name + "': frame counts differ");
        if (Lo.is_image_token64 && (Lo.batch_size % 64u != 0u || c.type == K44CmdType::S2D_2X2))
            throw std::runtime_error("command '" + c.name +
                                     "': not defined on the 64-frame interleaved layout");
        ax.type = c.type;
        ax.name = c.name;
        ax.y_off = c.y_off;
        ax.src_off = c.src_off;
        ax.pin = plane_of(Li);
        ax.pout = plane_of(Lo);
        uint32_t cin_planes = 0, cout_planes = 0;
        switch (c.type) {
        case K44CmdType::S2D_2X2:
            ax.C = c.Cin;
            cin_planes = c.Cin;
            cout_planes = 4u * c.Cin;
            if (2u * Lo.H > Li.H + 1u || 2u * Lo.W > Li.W + 1u)
                throw std::runtime_error("command '" + c.name + "': S2D output too large");
            break;
        case K44CmdType::MAXPOOL_2X2:
            ax.C = c.Cin;
            cin_planes = cout_planes = c.Cin;
            if (2u * Lo.H > Li.H || 2u * Lo.W > Li.W)
                throw std::runtime_error("command '" + c.name + "': pool output too large");
            break;
        case K44CmdType::MAXPOOL_5X5:
            ax.C = c.Cin;
            cin_planes = cout_planes = c.Cin;
            if (Lo.H != Li.H || Lo.W != Li.W)
                throw std::runtime_error("command '" + c.name + "': 5x5 pool changes the size");
            break;
        case K44CmdType::UPSAMPLE_2X:
            ax.C = c.Cin;
            cin_planes = cout_planes = c.Cin;
            if (Lo.H != 2u * Li.H || Lo.W != 2u * Li.W)
                throw std::runtime_error("command '" + c.name + "': upsample sizes");
            break;
        case K44CmdType::SCATTER_UP2X2:
            ax.C = c.Cout;
            ax.D = c.Cin / 4u;  // channels between quad plane groups
            if (c.Cin % 4u != 0u || ax.D < c.Cout)
                throw std::runtime_error("command '" + c.name + "': quad tensor channels");
            cin_planes = c.Cin;
            cout_planes = c.Cout;
            if (Lo.H != 2u * Li.H || Lo.W != 2u * Li.W)
                throw std::runtime_error("command '" + c.name + "': scatter-upconv sizes");
            break;
        default:
            throw std::runtime_error("command '" + c.name + "': not a spatial command");
        }
        ax.out_channels = cout_planes;
        const uint64_t n_canvas = plan_meta.canvas_elems;
        if (ax.src_off + (uint64_t)cin_planes * Li.channel_stride > n_canvas ||
            ax.y_off + (uint64_t)cout_planes * Lo.channel_stride > n_canvas)
            throw std::runtime_error("command '" + c.name + "': tensor past the canvas");
    }

    void build_aux(const K44ExecCmd &c, AuxExec &ax) {
        if (c.type == K44CmdType::S2D_2X2 || c.type == K44CmdType::MAXPOOL_2X2 ||
            c.type == K44CmdType::MAXPOOL_5X5 || c.type == K44CmdType::UPSAMPLE_2X ||
            c.type == K44CmdType::SCATTER_UP2X2) {
            build_spatial(c, ax);
            return;
        }
        const K44ResDesc &L = plan_meta.res_map.at(c.res_key_out);
        if (!L.is_1d_tokens)
            throw std::runtime_error("command '" + c.name + "': needs a 1-D token layout");
        ax.type = c.type;
        ax.name = c.name;
        ax.y_off = c.y_off;
        ax.src_off = c.src_off;
        ax.src2_off = c.src2_off;
        ax.stride = L.channel_stride;
        ax.tokens = L.W;
        ax.eps = c.eps;
        const uint64_t n_canvas = plan_meta.canvas_elems;
        auto need = [&](uint64_t off, uint64_t n, const char *what) {
            if (off > n_canvas || n > n_canvas - off)
                throw std::runtime_error("command '" + c.name + "': " + what + " past the canvas");
        };
        auto upload_f16 = [&](DevBuf<__half> &buf, const std::vector<uint16_t> &v) {
            std::vector<__half> h(v.size());
            std::memcpy(h.data(), v.data(), v.size() * 2u);
            buf.upload(h);
        };
        if (ax.stride % 64u != 0u) throw std::runtime_error("command '" + c.name + "': stride");
        switch (c.type) {
        case K44CmdType::RMSNORM_1D:
            ax.D = c.Cin;
            need(ax.src_off, (uint64_t)ax.D * ax.stride, "input");
            need(ax.y_off, (uint64_t)ax.D * ax.stride, "output");
            if (!c.gamma_folded) {
                if (c.h_bias.size() < ax.D) throw std::runtime_error("RMSNorm gamma too short");
                upload_f16(ax.table, std::vector<uint16_t>(c.h_bias.begin(), c.h_bias.begin() + ax.D));
            }
            break;
        case K44CmdType::SWIGLU_MUL_1D:
            ax.D = c.Cout;
            need(ax.src_off, (uint64_t)ax.D * ax.stride, "gate");
            need(ax.src2_off, (uint64_t)ax.D * ax.stride, "up");
            need(ax.y_off, (uint64_t)ax.D * ax.stride, "output");
            break;
        case K44CmdType::TOKEN_SHIFT_1D:
            ax.D = c.Cin;
            ax.rf = c.rf;
            ax.seq_len = c.seq_len;
            ax.decode = c.decode_state;
            ax.has_state = c.rf >= 2u;
            ax.state_off = c.state_off;
            need(ax.src_off, (uint64_t)ax.D * ax.stride, "input");
            need(ax.y_off, (uint64_t)ax.D * ax.stride, "output");
            if (ax.has_state) need(ax.state_off, (uint64_t)ax.D * (ax.rf - 1u) * 64u, "state");
            if (ax.decode ? ax.tokens > 64u : (ax.tokens % ax.seq_len != 0u ||
                                               ax.tokens / ax.seq_len > 64u))
                throw std::runtime_error("command '" + c.name +
                                         "': token shift supports at most 64 requests of equal length");
            if (c.h_table.size() != (size_t)ax.D * ax.rf)
                throw std::runtime_error("command '" + c.name + "': mix table size");
            upload_f16(ax.table, c.h_table);
            break;
        case K44CmdType::EMBED_1D:
            ax.D = c.Cout;
            ax.vocab = c.Cin;
            need(ax.y_off, (uint64_t)ax.D * ax.stride, "output");
            if (c.h_table.size() != (size_t)ax.D * ax.vocab)
                throw std::runtime_error("command '" + c.name + "': embedding table size");
            upload_f16(ax.table, c.h_table);
            id_tokens = std::max(id_tokens, ax.tokens);
            break;
        case K44CmdType::ARGMAX_1D:
            ax.D = c.Cin;
            need(ax.src_off, (uint64_t)ax.D * ax.stride, "input");
            id_tokens = std::max(id_tokens, ax.tokens);
            scratch_need = std::max(scratch_need, k44dev::argmax_scratch_floats(ax.D, ax.stride));
            break;
        default:
            throw std::runtime_error(std::string("command '") + c.name + "' of type " +
                                     cmd_type_str(c.type) + " is not supported by this executor");
        }
    }

    // whole: whole-plan execution (folded / fused commands apply).
    void launch_aux(const AuxExec &a, bool whole = false) {
        __half *cv = canvas.p;
        switch (a.type) {
        case K44CmdType::RMSNORM_1D:
            if (whole && a.shift_with != SIZE_MAX) {
                const AuxExec &t = *aux[a.shift_with];
                const k44dev::RmsShift sh{cv + t.y_off, t.table.p,
                                          t.has_state ? cv + t.state_off : nullptr, t.rf, 0u,
                                          t.decode ? 0u : t.seq_len};
                const float *inv = a.norm_fold != SIZE_MAX ? norm_invs.p + a.norm_fold * 64u : nullptr;
                K44_HIP(k44dev::launch_rmsnorm(cv + a.y_off, cv + a.src_off, a.table.p, a.D,
                                               a.stride, a.tokens, a.eps, stream, &sh, inv));
            } else if (whole && a.norm_fold != SIZE_MAX) {
                K44_HIP(k44dev::launch_rmsnorm(cv + a.y_off, cv + a.src_off, a.table.p, a.D,
                                               a.stride, a.tokens, a.eps, stream, nullptr,
                                               norm_invs.p + a.norm_fold * 64u));
            } else {
                K44_HIP(k44dev::launch_rmsnorm(cv + a.y_off, cv + a.src_off, a.table.p, a.D,
                                               a.stride, a.tokens, a.eps, stream));
            }
            break;
        case K44CmdType::SWIGLU_MUL_1D:
            if (whole && a.chain_inner != SIZE_MAX) {
                const AuxExec &in = *aux[a.chain_inner];
                K44_HIP(k44dev::launch_mul3(cv + a.y_off, cv + a.chain_other, cv + in.src_off,
                                            cv + in.src2_off, (uint64_t)a.D * a.stride, stream));
            } else {
                K44_HIP(k44dev::launch_mul(cv + a.y_off, cv + a.src_off, cv + a.src2_off,
                                           (uint64_t)a.D * a.stride, stream));
            }
            break;
        case K44CmdType::TOKEN_SHIFT_1D:
            K44_HIP(k44dev::launch_token_shift(cv + a.y_off, cv + a.src_off, a.table.p,
                                               a.has_state ? cv + a.state_off : nullptr, a.D,
                                               a.stride, a.tokens, a.rf, a.seq_len,
                                               a.decode ? 1 : 0, stream));
            break;
        case K44CmdType::EMBED_1D:
            K44_HIP(k44dev::launch_embed(cv + a.y_off, a.table.p, ids.p, a.D, a.vocab, a.stride,
                                         a.tokens, stream));
            break;
        case K44CmdType::S2D_2X2:
            K44_HIP(k44dev::launch_s2d(cv + a.y_off, cv + a.src_off, a.C, a.pin, a.pout, stream));
            K44_HIP(k44dev::launch_halo_clear(cv + a.y_off, a.out_channels, a.pout, stream));
            break;
        case K44CmdType::MAXPOOL_2X2:
            K44_HIP(k44dev::launch_maxpool2(cv + a.y_off, cv + a.src_off, a.C, a.pin, a.pout, stream));
            K44_HIP(k44dev::launch_halo_clear(cv + a.y_off, a.out_channels, a.pout, stream));
            break;
        case K44CmdType::MAXPOOL_5X5:
            K44_HIP(k44dev::launch_maxpool5(cv + a.y_off, cv + a.src_off, a.C, a.pin, a.pout, stream));
            K44_HIP(k44dev::launch_halo_clear(cv + a.y_off, a.out_channels, a.pout, stream));
            break;
        case K44CmdType::UPSAMPLE_2X:
            K44_HIP(k44dev::launch_upsample2(cv + a.y_off, cv + a.src_off, a.C, a.pin, a.pout, stream));
            K44_HIP(k44dev::launch_halo_clear(cv + a.y_off, a.out_channels, a.pout, stream));
            break;
        case K44CmdType::SCATTER_UP2X2:
            K44_HIP(k44dev::launch_scatter_up2(cv + a.y_off, cv + a.src_off, a.C, a.D, a.pin,
                                               a.pout, stream));
            K44_HIP(k44dev::launch_halo_clear(cv + a.y_off, a.out_channels, a.pout, stream));
            break;
        case K44CmdType::ARGMAX_1D:
            K44_HIP(k44dev::launch_argmax(ids.p, hist_steps ? history.p : nullptr, step_ctr.p,
                                          hist_steps, cv + a.src_off, a.D, a.stride, a.tokens,
                                          scratch.p, stream));
            break;
        default:
            throw std::runtime_error("unsupported aux command");
        }
    }

    void init(const K44WavePlan &plan) {
        {
            const int xo = tune(Tune::XcdOrder);
            xcd_order = xo < 0 ? 2u : (uint32_t)std::min(xo, 2);
        }
        free_all();
        plan_meta.res_map = plan.res_map;
        plan_meta.canvas_elems = plan.canvas_elems;
        plan_meta.input_off = plan.input_off;
        plan_meta.input_c = plan.input_c;
        plan_meta.input_h = plan.input_h;
        plan_meta.input_w = plan.input_w;
        plan_meta.input_res_key = plan.input_res_key;
        plan_meta.output_off = plan.output_off;
        plan_meta.output_c = plan.logical_output_c;
        plan_meta.output_h = plan.output_h;
        plan_meta.output_w = plan.output_w;
        plan_meta.output_res_key = plan.output_res_key;
        plan_meta.batch_size = plan.batch_size;
        for (const auto &c : plan.cmds) {
            if (c.type == K44CmdType::K44_WAVE) {
                auto wx = std::make_unique<WaveExec>();
                build_wave(c, *wx);
                wave_cmd.push_back(ops.size());
                ops.push_back({true, waves.size()});
                waves.push_back(std::move(wx));
            } else {
                auto ax = std::make_unique<AuxExec>();
                build_aux(c, *ax);
                aux_cmd.push_back(ops.size());
                ops.push_back({false, aux.size()});
                aux.push_back(std::move(ax));
            }
        }
        fuse_products();
        fuse_mul_chains();
        fuse_norm_shifts();
        fuse_norms();
        form_runs();
        K44_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
        K44_HIP(hipEventCreate(&ev0));
        K44_HIP(hipEventCreate(&ev1));
        canvas.alloc((plan.canvas_elems + kCanvasSlack + 63u) / 64u * 64u + fold_elems);
        if (scratch_need) scratch.alloc(scratch_need);
        {
            size_t n_arrive = 0;
            for (auto &wp : waves)
                if (wp->reduce_in_kernel) {
                    wp->arrive_off = n_arrive;
                    n_arrive += wp->rows;
                }
            if (n_arrive) {
                arrive.alloc(n_arrive);
                K44_HIP(hipMemsetAsync(arrive.p, 0, n_arrive * sizeof(uint32_t), stream));
            }
        }
        if (!norm_folds.empty()) {
            const NormFold &last = norm_folds.back();
            const size_t slots = last.slot0 + last.tiles;
            norm_slots.alloc(slots * 64u);
            norm_ctrs.alloc(norm_folds.size());
            norm_invs.alloc(norm_folds.size() * 64u);
            K44_HIP(hipMemsetAsync(norm_slots.p, 0, slots * 64u * sizeof(uint32_t), stream));
            K44_HIP(hipMemsetAsync(norm_ctrs.p, 0, norm_folds.size() * sizeof(uint32_t), stream));
            K44_HIP(hipMemsetAsync(norm_invs.p, 0, norm_folds.size() * 64u * sizeof(float), stream));
        }
        upload_mfma_descriptors();
        K44_HIP(hipMemsetAsync(canvas.p, 0,
                               ((plan.canvas_elems + kCanvasSlack + 63u) / 64u * 64u + fold_elems) * 2u,
                               stream));
        if (id_tokens) {
            ids.alloc(id_tokens);
            step_ctr.alloc(1);
            K44_HIP(hipMemsetAsync(ids.p, 0, id_tokens * 4u, stream));
            K44_HIP(hipMemsetAsync(step_ctr.p, 0, 4u, stream));
        }
        K44_HIP(hipStreamSynchronize(stream));
        build_program();
        build_report();
        initialized = true;
    }

    // Canvas ranges an aux command reads and writes (the 2-D commands: everything).
    void aux_ranges(const AuxExec &a, Ranges &rd, Ranges &wr) const {
        const uint64_t n = (uint64_t)a.D * a.stride;
        rd.clear();
        wr.clear();
        switch (a.type) {
        case K44CmdType::RMSNORM_1D:
            rd = {{a.src_off, a.src_off + n}};
            wr = {{a.y_off, a.y_off + n}};
            break;
        case K44CmdType::SWIGLU_MUL_1D:
            rd = merge_ranges({{a.src_off, a.src_off + n}, {a.src2_off, a.src2_off + n}});
            wr = {{a.y_off, a.y_off + n}};
            break;
        case K44CmdType::TOKEN_SHIFT_1D: {
            Ranges r = {{a.src_off, a.src_off + n}}, w = {{a.y_off, a.y_off + n}};
            if (a.has_state) {
                const uint64_t ns = (uint64_t)a.D * (a.rf - 1u) * 64u;
                r.push_back({a.state_off, a.state_off + ns});
                w.push_back({a.state_off, a.state_off + ns});
            }
            rd = merge_ranges(std::move(r));
            wr = merge_ranges(std::move(w));
            break;
        }
        case K44CmdType::EMBED_1D:
            wr = {{a.y_off, a.y_off + n}};
            break;
        case K44CmdType::ARGMAX_1D:
            rd = {{a.src_off, a.src_off + n}};
            break;
        default:
            rd = wr = {{0u, UINT64_MAX}};
        }
    }

    // Element-wise multiplies (SWIGLU_MUL_1D) whose product is read only by narrow MFMA waves
    // of 64 / 128-neuron tiles are folded into those waves' gathers: the wave loads the
    // operands' rows and multiplies with the commands' own rounding (y = fp16(a*b); a chain
    // m = q*(k*v) as fp16(q*fp16(k*v))), so its input and output are bit-identical and two
    // launches fewer run per chain.  Conditions, from the canvas ranges of the commands in plan
    // order: the product is not the plan output; every reader until it is overwritten is such a
    // wave reading it only as gather input (an inner product: exactly one reader, the outer
    // multiply); every operand stays intact from the first folded multiply through the last
    // reader — or, when the canvas allocator has reused its range in between (the plan only
    // needed it until the multiply), the operand is relocated: the MFMA waves that produce it
    // (the sub-waves of one projection, together covering every row) write it to a private
    // region past the canvas instead, provided nothing but the folded multiplies reads it.
    // Whole-plan execution only: execute_range runs every command as compiled.
    // Tuning switch fuse=0 disables it.
    void fuse_products() {
        if (tune(Tune::Fuse) == 0) return;
        const size_t n = ops.size();
        std::vector<Ranges> rd(n), wr(n);
        for (size_t i = 0; i < n; ++i) {
            if (ops[i].first) {
                rd[i] = waves[ops[i].second]->rd;
                wr[i] = waves[ops[i].second]->wr;
            } else {
                aux_ranges(*aux[ops[i].second], rd[i], wr[i]);
            }
        }
        Ranges out_rng = {{0u, UINT64_MAX}};
        {
            auto it = plan_meta.res_map.find(plan_meta.output_res_key);
            if (it != plan_meta.res_map.end())
                out_rng = {{plan_meta.output_off,
                            plan_meta.output_off +
                                (uint64_t)plan_meta.output_c * it->second.channel_stride}};
        }
        typedef std::pair<uint64_t, uint64_t> Rng;
        auto is_mul = [&](size_t i) {
            return !ops[i].first && aux[ops[i].second]->type == K44CmdType::SWIGLU_MUL_1D;
        };
        auto covers = [](const Ranges &a, const Rng &r) {
            for (const auto &x : a)
                if (x.first <= r.first && r.second <= x.second) return true;
            return false;
        };
        auto inside = [](const Ranges &a, const Rng &r) {
            for (const auto &x : a)
                if (x.first < r.first || x.second > r.second) return false;
            return true;
        };
        // Readers of the tensor in range R written by op i, up to the first op that writes into
        // R (the compiler's allocator reuses a range only once its tensor is dead); false if the
        // tensor is still alive at the end of the plan and overlaps the plan output.
        auto readers = [&](size_t i, Rng R, std::vector<size_t> &out) {
            const Ranges rr = {R};
            for (size_t j = i + 1; j < n; ++j) {
                if (ranges_overlap(rd[j], rr)) out.push_back(j);
                if (ranges_overlap(wr[j], rr)) return true;
            }
            return !ranges_overlap(rr, out_rng);
        };
        auto out_range = [&](size_t i) {
            const AuxExec &a = *aux[ops[i].second];
            return Rng(a.y_off, a.y_off + (uint64_t)a.D * a.stride);
        };
        auto opnd_range = [&](size_t i, int k) {
            const AuxExec &a = *aux[ops[i].second];
            const uint64_t o = k == 0 ? a.src_off : a.src2_off;
            return Rng(o, o + (uint64_t)a.D * a.stride);
        };
        const uint64_t fold_base = (plan_meta.canvas_elems + kCanvasSlack + 63u) / 64u * 64u;
        auto note = [&](size_t i, const char *why) {
            aux[ops[i].second]->fuse_note = why;
        };
        for (size_t i = 0; i < n; ++i) {
            if (!is_mul(i) || aux[ops[i].second]->fused) continue;
            const auto R = out_range(i);
            const uint64_t D = aux[ops[i].second]->D, stride = aux[ops[i].second]->stride;
            std::vector<size_t> rds;
            if (!readers(i, R, rds) || rds.empty()) {
                note(i, "product is the plan output or unread");
                continue;
            }
            bool ok = true;
            for (size_t j : rds) {
                if (!ops[j].first) {
                    ok = false;
                    break;
                }
                const WaveExec &w = *waves[ops[j].second];
                ok = w.mfma && w.narrow && (w.cluster == 64u || w.cluster == 128u) &&
                     !w.tile2d && !w.xprod;
                for (const auto &x : w.xrd) ok = ok && R.first <= x.first && x.second <= R.second;
                // residual rows must not read the product (only the gather is replaced)
                ok = ok && !ranges_overlap(w.resrd, Ranges{R});
                if (!ok) break;
            }
            if (!ok) {
                note(i, "a reader is not a narrow 64/128-neuron wave gathering only the product");
                continue;
            }
            // Operands; an operand produced by a multiply read only here is expanded (3 leaves).
            Rng leaf[3];
            int nleaf = 2;
            leaf[0] = opnd_range(i, 0);
            leaf[1] = opnd_range(i, 1);
            size_t inner = n;
            for (int k = 0; k < 2 && inner == n; ++k) {
                const auto Q = opnd_range(i, k);
                for (size_t p = i; p-- > 0;) {
                    if (!ranges_overlap(wr[p], Ranges{Q})) continue;
                    if (is_mul(p) && !aux[ops[p].second]->fused && out_range(p) == Q) {
                        std::vector<size_t> r2;
                        if (readers(p, Q, r2) && r2.size() == 1u && r2[0] == i) {
                            inner = p;
                            leaf[0] = opnd_range(i, 1 - k);  // A: the other operand
                            leaf[1] = opnd_range(p, 0);
                            leaf[2] = opnd_range(p, 1);
                            nleaf = 3;
                        }
                    }
                    break;
                }
            }
            const size_t first = inner < n ? inner : i;
            auto chain_mul = [&](size_t j) { return j == i || j == inner; };
            // Each operand: intact in place, or relocatable (its producers found and only the
            // chain's multiplies read it).
            std::vector<size_t> prods[3];
            bool move[3] = {false, false, false};
            for (int k = 0; k < nleaf && ok; ++k) {
                const Rng L = leaf[k];
                bool intact = true;
                for (size_t j = first + 1; j <= rds.back() && intact; ++j)
                    if (!chain_mul(j)) intact = !ranges_overlap(wr[j], Ranges{L});
                if (intact) continue;
                // Producers: MFMA waves writing inside L, back from the chain, until their rows
                // cover all D rows of L.
                Ranges cov;
                bool full = false;
                for (size_t p = first; p-- > 0 && !full;) {
                    if (!ranges_overlap(wr[p], Ranges{L})) continue;
                    if (!ops[p].first) break;
                    const WaveExec &w = *waves[ops[p].second];
                    if (!w.mfma || w.tile2d || !inside(w.wr, L)) break;
                    prods[k].push_back(p);
                    for (const auto &x : w.wr) cov.push_back(x);
                    cov = merge_ranges(std::move(cov));
                    full = true;
                    for (uint64_t r = 0; r < D && full; ++r)
                        full = covers(cov, Rng(L.first + r * stride, L.first + r * stride + 1u));
                }
                ok = full;
                if (!ok) {
                    note(i, "operand overwritten in place and its producers not relocatable");
                    break;
                }
                // Nothing but the producers before the chain and the chain's multiplies after
                // the last producer reads L while it is alive.
                const size_t p0 = prods[k].back(), p1 = prods[k].front();
                for (size_t j = p0; j < first && ok; ++j) {
                    bool is_prod = false;
                    for (size_t q : prods[k]) is_prod = is_prod || q == j;
                    if (!is_prod) ok = !ranges_overlap(rd[j], Ranges{L});
                }
                std::vector<size_t> lr;
                ok = ok && readers(p1, L, lr);
                for (size_t j : lr) ok = ok && chain_mul(j);
                if (!ok) note(i, "relocatable operand has other readers");
                move[k] = true;
            }
            if (!ok) continue;
            note(i, nleaf == 3 ? "folded (3 operands)" : "folded (2 operands)");
            // Apply: relocate operands, skip the multiplies, point the readers' gathers.
            uint64_t at[3];
            for (int k = 0; k < nleaf; ++k) {
                at[k] = leaf[k].first;
                if (!move[k]) continue;
                at[k] = fold_base + fold_elems;
                fold_elems += D * stride;
                for (size_t p : prods[k]) {
                    WaveExec &w = *waves[ops[p].second];
                    const uint64_t delta = at[k] - leaf[k].first;
                    w.y_off_run = w.y_off + delta;
                    Ranges m;
                    for (const auto &x : w.wr) m.push_back({x.first + delta, x.second + delta});
                    w.wr_run = merge_ranges(std::move(m));
                    w.why += "; output relocated for a folded multiply";
                }
            }
            aux[ops[i].second]->fused = true;
            if (inner < n) aux[ops[inner].second]->fused = true;
            for (size_t j : rds) {
                WaveExec &w = *waves[ops[j].second];
                w.xprod = (uint32_t)nleaf;
                Ranges fr = w.resrd;
                for (int k = 0; k < nleaf; ++k) {
                    w.xd[k] = (int64_t)at[k] - (int64_t)R.first;
                    for (const auto &x : w.xrd)
                        fr.push_back({(uint64_t)((int64_t)x.first + w.xd[k]),
                                      (uint64_t)((int64_t)x.second + w.xd[k])});
                }
                w.rd_run = merge_ranges(std::move(fr));
                w.why += nleaf == 3 ? "; gathers fp16(a*fp16(b*c)) (two multiplies folded)"
                                    : "; gathers fp16(a*b) (multiply folded)";
            }
        }
    }

    // Chains of element-wise multiplies left after fuse_products (prefill: m = q*(k*v) whose
    // readers are wide MFMA waves): an inner multiply whose product only the outer one reads is
    // not launched; the outer one computes fp16(other * fp16(b * c)) from the inner one's
    // operands in one pass (bit-identical, one launch and one tensor round trip fewer).
    // Conditions, from the canvas ranges in plan order: the inner operands stay intact from the
    // inner multiply through the outer one, and the output is either disjoint from each operand
    // or exactly one of them (then every element is read before it is written, by one thread).
    // Whole-plan execution only; tuning switch fuse=0 disables it.
    void fuse_mul_chains() {
        if (tune(Tune::Fuse) == 0) return;
        const size_t n = ops.size();
        std::vector<Ranges> rd(n), wr(n);
        for (size_t i = 0; i < n; ++i) {
            if (ops[i].first) {
                rd[i] = waves[ops[i].second]->rd_run;
                wr[i] = waves[ops[i].second]->wr_run;
            } else if (!aux[ops[i].second]->fused) {
                aux_ranges(*aux[ops[i].second], rd[i], wr[i]);
            }
        }
        Ranges out_rng = {{0u, UINT64_MAX}};
        {
            auto it = plan_meta.res_map.find(plan_meta.output_res_key);
            if (it != plan_meta.res_map.end())
                out_rng = {{plan_meta.output_off,
                            plan_meta.output_off +
                                (uint64_t)plan_meta.output_c * it->second.channel_stride}};
        }
        typedef std::pair<uint64_t, uint64_t> Rng;
        auto is_mul = [&](size_t i) {
            return !ops[i].first && aux[ops[i].second]->type == K44CmdType::SWIGLU_MUL_1D &&
                   !aux[ops[i].second]->fused && aux[ops[i].second]->chain_inner == SIZE_MAX;
        };
        auto rng = [&](size_t i, int k) {
            const AuxExec &a = *aux[ops[i].second];
            const uint64_t o = k == 0 ? a.src_off : k == 1 ? a.src2_off : a.y_off;
            return Rng(o, o + (uint64_t)a.D * a.stride);
        };
        for (size_t i = 0; i < n; ++i) {
            if (!is_mul(i)) continue;
            AuxExec &outer = *aux[ops[i].second];
            const Rng R = rng(i, 2);
            for (int k = 0; k < 2; ++k) {
                const Rng Q = rng(i, k);
                size_t p = n;
                for (size_t j = i; j-- > 0;)
                    if (ranges_overlap(wr[j], Ranges{Q})) {
                        p = j;
                        break;
                    }
                if (p == n || !is_mul(p) || rng(p, 2) != Q) continue;
                const AuxExec &in = *aux[ops[p].second];
                if (in.D != outer.D || in.stride != outer.stride) continue;
                // the product q: read by the outer multiply only until overwritten, and not the
                // plan output if nothing overwrites it
                bool ok = true, overwritten = false;
                for (size_t j = p + 1; j < n && ok && !overwritten; ++j) {
                    if (j != i && ranges_overlap(rd[j], Ranges{Q})) ok = false;
                    overwritten = ranges_overlap(wr[j], Ranges{Q});
                }
                ok = ok && (overwritten || !ranges_overlap(Ranges{Q}, out_rng));
                const Rng A = rng(i, 1 - k), B = rng(p, 0), C = rng(p, 1);
                for (size_t j = p + 1; j < i && ok; ++j)
                    ok = !ranges_overlap(wr[j], Ranges{B}) && !ranges_overlap(wr[j], Ranges{C});
                for (const Rng &X : {A, B, C})
                    ok = ok && (X == R || !ranges_overlap(Ranges{X}, Ranges{R}));
                if (!ok) continue;
                aux[ops[p].second]->fused = true;
                aux[ops[p].second]->fuse_note = "run by the multiply that reads it (3-operand kernel)";
                outer.chain_inner = ops[p].second;
                outer.chain_other = A.first;
                outer.fuse_note = "runs the inner multiply it reads (3-operand kernel)";
                rd[p].clear();
                wr[p].clear();
                rd[i] = merge_ranges({A, B, C});
                break;
            }
        }
    }

    // An RMSNorm followed directly by the token shift of its output runs the shift in the same
    // kernel (whole-plan execution; bit-identical to the two commands).  Decode: the norm's
    // decode form keeps one channel per thread, so the shift of that channel's tokens follows
    // in place.  Prefill (the register-resident 32-token form): each workgroup also normalizes
    // the 4 tokens before its block (RF - 1 <= 4) and shifts its own tokens
    // (k44_rmsnorm_shift_prefill_kernel).
    // Tuning switch fuse=0 keeps both launches.
    void fuse_norm_shifts() {
        if (tune(Tune::Fuse) == 0) return;
        for (size_t i = 0; i + 1u < ops.size(); ++i) {
            if (ops[i].first || ops[i + 1u].first) continue;
            AuxExec &N = *aux[ops[i].second];
            AuxExec &T = *aux[ops[i + 1u].second];
            if (N.type != K44CmdType::RMSNORM_1D || T.type != K44CmdType::TOKEN_SHIFT_1D ||
                N.fused || T.fused || T.src_off != N.y_off || T.D != N.D ||
                T.stride != N.stride || T.tokens != N.tokens || T.rf == 0u || T.rf > 9u)
                continue;
            if (T.decode) {
                if (N.stride != 64u || N.tokens == 0u || N.tokens > 64u ||
                    (T.rf > 1u && !T.has_state))
                    continue;
                // The launcher's decode geometry must give one channel per thread.
                const uint32_t chunks = (N.tokens + 7u) / 8u;
                uint32_t slices = (256u + chunks - 1u) / chunks;
                slices = std::min(slices, (N.D + 255u) / 256u);
                if ((N.D + slices - 1u) / slices > 256u) continue;
            } else if (!k44dev::rmsnorm_shift_prefill_ok(N.D, N.stride, N.tokens, T.rf,
                                                         T.seq_len)) {
                continue;
            }
            // Every workgroup of the fused kernel reads all D rows of the norm's input for its
            // sums while other workgroups already store shift outputs and state: the canvas
            // allocator may have given the input's range (dead after the norm) to the shift's
            // output, so fuse only when the shift writes nothing the norm reads.
            Ranges rd_n, wr_n, rd_t, wr_t;
            aux_ranges(N, rd_n, wr_n);
            aux_ranges(T, rd_t, wr_t);
            if (ranges_overlap(wr_t, rd_n)) continue;
            // The prefill form also reads the 4 tokens before each workgroup's block: the norm
            // must not write over its own input either.
            if (!T.decode && ranges_overlap(wr_n, rd_n)) continue;
            N.shift_with = ops[i + 1u].second;
            T.fused = true;
        }
    }

    // RMSNorms of decode-sized plans whose input is written by narrow 64/128-neuron MFMA waves
    // (the sub-waves of the projections before them, each tile's outputs stored by one
    // workgroup) take their per-token scales from those waves: every producer tile adds the
    // exact sums of squares of the values it stored, and the last tile of the tensor forms the
    // scales (k44_mfma_narrow.hip, narrow_norm_publish).  The sums are exact, so the scales equal
    // the norm kernel's own bit for bit.  A norm read only by narrow 64/128-neuron waves gathering
    // it plainly is then not launched: those waves gather its input and normalise it in the
    // gather with the kernel's expression (xprod 4).  Otherwise (a norm that runs the decode
    // token shift) the norm kernel runs with the scales and skips its sum pass.  Conditions, from
    // the canvas ranges of the commands in plan order: the producers are the last writers of
    // the input, together write each of its D rows exactly once, and run their whole epilogue
    // in one workgroup per tile (unsplit, or split-K reduced in the launch); for the consumers,
    // the input stays intact until the last of them, and the norm's output is not the plan
    // output.  Whole-plan execution only; tuning switch fuse=0 disables it.
    void fuse_norms() {
        if (tune(Tune::Fuse) == 0) return;
        const size_t n = ops.size();
        std::vector<Ranges> rd(n), wr(n);
        for (size_t i = 0; i < n; ++i) {
            if (ops[i].first) {
                rd[i] = waves[ops[i].second]->rd_run;
                wr[i] = waves[ops[i].second]->wr_run;
            } else if (!aux[ops[i].second]->fused) {
                const AuxExec &A = *aux[ops[i].second];
                aux_ranges(A, rd[i], wr[i]);
                if (A.shift_with != SIZE_MAX) {  // the shift it runs
                    Ranges r2, w2;
                    aux_ranges(*aux[A.shift_with], r2, w2);
                    for (const auto &x : r2) rd[i].push_back(x);
                    for (const auto &x : w2) wr[i].push_back(x);
                    rd[i] = merge_ranges(std::move(rd[i]));
                    wr[i] = merge_ranges(std::move(wr[i]));
                }
            }
        }
        Ranges out_rng = {{0u, UINT64_MAX}};
        {
            auto it = plan_meta.res_map.find(plan_meta.output_res_key);
            if (it != plan_meta.res_map.end())
                out_rng = {{plan_meta.output_off,
                            plan_meta.output_off +
                                (uint64_t)plan_meta.output_c * it->second.channel_stride}};
        }
        typedef std::pair<uint64_t, uint64_t> Rng;
        auto narrow_long = [&](const WaveExec &w) {
            return w.mfma && w.narrow && (w.cluster == 64u || w.cluster == 128u) && !w.tile2d;
        };
        for (size_t i = 0; i < n; ++i) {
            if (ops[i].first) continue;
            AuxExec &N = *aux[ops[i].second];
            if (N.type != K44CmdType::RMSNORM_1D || N.fused || N.tokens == 0u || N.tokens > 16u ||
                N.D == 0u || N.D > 65536u || N.stride == 0u || (N.stride & (N.stride - 1u)) ||
                N.stride > 64u)
                continue;
            const Rng X(N.src_off, N.src_off + (uint64_t)N.D * N.stride);
            const Rng Y(N.y_off, N.y_off + (uint64_t)N.D * N.stride);
            // producers: walking back, every writer into X until each row is covered
            std::vector<size_t> prods;
            std::vector<uint8_t> row_seen(N.D, 0u);
            uint32_t covered = 0;
            bool ok = true;
            for (size_t p = i; p-- > 0 && ok && covered < N.D;) {
                if (!ranges_overlap(wr[p], Ranges{X})) continue;
                if (!ops[p].first) {
                    ok = false;
                    break;
                }
                const WaveExec &w = *waves[ops[p].second];
                ok = narrow_long(w) && (w.kgroups <= 1u || w.reduce_in_kernel) &&
                     w.y_off_run == w.y_off;
                for (const auto &x : w.wr_run) {
                    if (!ok) break;
                    // rows of X from their first element (merged ranges span consecutive
                    // rows); each row written once, at least its first N.tokens columns
                    ok = x.first >= X.first && x.second <= X.second &&
                         (x.first - X.first) % N.stride == 0u;
                    if (!ok) break;
                    const uint64_t r0 = (x.first - X.first) / N.stride;
                    const uint64_t r1 = (x.second - X.first + N.stride - 1u) / N.stride;
                    ok = (x.second - X.first) - (r1 - 1u) * N.stride >= N.tokens;
                    for (uint64_t r = r0; r < r1 && ok; ++r) {
                        ok = !row_seen[r];
                        row_seen[r] = 1u;
                        ++covered;
                    }
                }
                if (ok) prods.push_back(ops[p].second);
            }
            if (!ok || covered != N.D || prods.empty()) continue;
            // consumers (a norm without a fused shift): readers of Y until overwritten
            std::vector<size_t> cons;
            bool consume = N.shift_with == SIZE_MAX;
            if (consume) {
                size_t last = i;
                bool overwritten = false;
                for (size_t j = i + 1; j < n && consume && !overwritten; ++j) {
                    if (ranges_overlap(rd[j], Ranges{Y})) {
                        if (!ops[j].first) {
                            consume = false;
                            break;
                        }
                        const WaveExec &w = *waves[ops[j].second];
                        consume = narrow_long(w) && w.xprod == 0u &&
                                  !ranges_overlap(w.resrd, Ranges{Y});
                        for (const auto &x : w.xrd)
                            consume = consume && Y.first <= x.first && x.second <= Y.second;
                        cons.push_back(ops[j].second);
                        last = j;
                    }
                    overwritten = ranges_overlap(wr[j], Ranges{Y});
                }
                consume = consume && !cons.empty() &&
                          (overwritten || !ranges_overlap(Ranges{Y}, out_rng));
                for (size_t j = i + 1; j <= last && consume; ++j)
                    consume = !ranges_overlap(wr[j], Ranges{X});
            }
            // fold
            NormFold f;
            f.norm = ops[i].second;
            f.slot0 = norm_folds.empty() ? 0u : norm_folds.back().slot0 + norm_folds.back().tiles;
            for (size_t pw : prods) {
                WaveExec &w = *waves[pw];
                w.norm_fold = norm_folds.size();
                w.norm_tile0 = f.tiles;
                f.tiles += w.rows;
                w.why += "; its tiles form the sums of squares of a folded RMSNorm";
            }
            f.consumers = consume;
            N.norm_fold = norm_folds.size();
            if (consume) {
                N.fused = true;
                N.fuse_note = "folded: scales formed by its producers, rows normalised in its "
                              "readers' gathers";
                for (size_t cw : cons) {
                    WaveExec &w = *waves[cw];
                    w.xprod = 4u;
                    w.xnorm = norm_folds.size();
                    w.xd[0] = (int64_t)X.first - (int64_t)Y.first;
                    Ranges fr = w.resrd;
                    for (const auto &x : w.xrd)
                        fr.push_back({(uint64_t)((int64_t)x.first + w.xd[0]),
                                      (uint64_t)((int64_t)x.second + w.xd[0])});
                    w.rd_run = merge_ranges(std::move(fr));
                    w.why += "; gathers its input through a folded RMSNorm";
                }
            } else {
                N.fuse_note = "scales formed by its producers (no sum pass)";
            }
            norm_folds.push_back(f);
        }
    }

    // Plan order -> runs: consecutive MFMA waves of one kernel configuration join a group while
    // no member writes what another reads or writes (checked on canvas element ranges).
    void form_runs() {
        const bool grouping = tune(Tune::Group) != 0;
        runs.clear();
        groups.clear();
        for (const auto &op : ops) {
            if (!op.first) {
                if (!aux[op.second]->fused) runs.push_back({0, op.second});
                continue;
            }
            const WaveExec &w = *waves[op.second];
            scratch_need = std::max(scratch_need, w.part_floats);
            if (!w.mfma || w.tile2d) {  // 2-D waves: launched alone, halo clear after each
                runs.push_back({1, op.second});
                continue;
            }
            // Join the latest group of the same kernel configuration among the last group
            // launches before this wave, provided the wave is independent of every member of
            // that group and of the groups after it: it then runs earlier than in plan order
            // with the same inputs (the groups in between neither write what it reads nor read
            // or write what it writes).  Projections whose sub-waves take different kernels
            // (paired full-pattern tiles, single union tiles) thus still share launches.
            bool joined = false;
            for (size_t ri = runs.size(), seen = 0; grouping && ri-- > 0 && seen < 8u; ++seen) {
                if (runs[ri].first != 2) break;
                MfmaGroupExec &g = *groups[runs[ri].second];
                bool indep = true;
                for (size_t m : g.members) {
                    const WaveExec &o = *waves[m];
                    indep = !ranges_overlap(w.wr_run, o.rd_run) &&
                            !ranges_overlap(w.rd_run, o.wr_run) &&
                            !ranges_overlap(w.wr_run, o.wr_run);
                    if (!indep) break;
                }
                if (!indep) break;
                if (g.nt == w.cluster && g.mt == w.mt && g.rows == w.rows_per_stage &&
                    g.dma == w.dma && g.stream_loads == w.stream_loads && g.dshape == w.dshape &&
                    g.prod == w.xprod && g.mis == w.mis && g.members.size() < 64u) {
                    g.members.push_back(op.second);
                    g.part_floats += w.part_floats;
                    joined = true;
                    break;
                }
            }
            if (!joined) {
                auto g = std::make_unique<MfmaGroupExec>();
                g->members = {op.second};
                g->nt = w.cluster;
                g->mt = w.mt;
                g->rows = w.rows_per_stage;
                g->dma = w.dma;
                g->mis = w.mis;
                g->stream_loads = w.stream_loads;
                g->dshape = w.dshape;
                g->prod = w.xprod;
                g->part_floats = w.part_floats;
                runs.push_back({2, groups.size()});
                groups.push_back(std::move(g));
            }
        }
        // Split-K is chosen per wave for parallelism; a group launch has the workgroups of all
        // its members, so a wide-token group that fills the GPU without splitting (>= 256
        // workgroups) runs unsplit: no partial planes, no epilogue kernel (config-5 prefill
        // 29.0 -> 27.0 ms).  Decode groups keep their split: measured 1.22 ms per step against
        // 1.46 ms unsplit — at 16 tokens the extra workgroups stream weights faster than the
        // epilogue costs.
        if (tune(Tune::GroupSplit) != 0) {
            for (auto &gp : groups) {
                MfmaGroupExec &g = *gp;
                if (g.mt == 16u) continue;
                uint64_t base = 0;
                for (size_t m : g.members) {
                    const WaveExec &w = *waves[m];
                    base += (uint64_t)w.rows * (w.tokens / w.mt);
                }
                if (base < 256u) continue;
                g.part_floats = 0;
                for (size_t m : g.members) {
                    WaveExec &w = *waves[m];
                    set_split(w, 1u);
                    g.part_floats += w.part_floats;
                }
            }
        }
        for (const auto &g : groups) scratch_need = std::max(scratch_need, g->part_floats);
    }

    // Contraction split of an MFMA wave into `want` chunks (k-steps for the narrow kernels,
    // stages of rows_per_stage positions otherwise).
    static void set_split(WaveExec &w, uint32_t want) {
        const uint32_t units = w.narrow ? w.ksteps : w.K * w.S / w.rows_per_stage;
        want = std::max(1u, std::min(want, units));
        w.stage_chunk = (units + want - 1u) / want;
        w.kgroups = (units + w.stage_chunk - 1u) / w.stage_chunk;
        w.part_floats = w.kgroups > 1u ? (size_t)w.kgroups * w.cout * w.part_tokens : 0u;
    }

    k44dev::MfmaTileArgs mfma_args(const WaveExec &w, float *part, bool fused) const {
        k44dev::MfmaTileArgs a{};
        if (fused && w.xprod) {
            a.xprod = w.xprod;
            for (int i = 0; i < 3; ++i) a.xd[i] = w.xd[i];
        }
        a.X = canvas.p;
        a.seg = w.seg.p;
        a.Wf = w.w.p;
        a.bias = w.bias.p;
        a.cmap = w.cmap.p;
        a.Y = canvas.p + (fused ? w.y_off_run : w.y_off);
        a.R = w.has_res ? canvas.p + w.res_off : nullptr;
        a.step = w.step;
        a.K = w.K;
        a.S = w.S;
        a.ksteps = w.ksteps;
        a.out_stride = w.out_stride;
        a.act = w.act;
        if (w.narrow)  // chunk in k-steps
            a.stage_chunk = w.kgroups > 1u ? w.stage_chunk : w.ksteps;
        else  // chunk in stages of rows_per_stage positions
            a.stage_chunk = w.kgroups > 1u ? w.stage_chunk : a.K * a.S / w.rows_per_stage;
        a.part = w.kgroups > 1u ? part : nullptr;
        if (fused && w.reduce_in_kernel) a.arrive = arrive.p + w.arrive_off;
        if (fused && w.norm_fold != SIZE_MAX) {
            const NormFold &f = norm_folds[w.norm_fold];
            const AuxExec &N = *aux[f.norm];
            a.norm_part = norm_slots.p + (f.slot0 + w.norm_tile0) * 64u;
            a.norm_all = norm_slots.p + f.slot0 * 64u;
            a.norm_cnt = norm_ctrs.p + w.norm_fold;
            a.norm_inv = norm_invs.p + w.norm_fold * 64u;
            a.norm_tiles = f.tiles;
            a.norm_D = N.D;
            a.norm_eps = N.eps;
        }
        if (fused && w.xnorm != SIZE_MAX) {
            const AuxExec &N = *aux[norm_folds[w.xnorm].norm];
            a.xinv = norm_invs.p + w.xnorm * 64u;
            a.xgamma = N.table.p;
            a.xg_base = N.y_off;
            uint32_t sh = 0;
            while ((1u << sh) < N.stride) ++sh;
            a.xg_shift = sh;
        }
        a.cout = w.cout;
        a.tokens = w.part_tokens;
        a.tiles = w.rows;
        a.ttiles = w.narrow ? 1u : w.tokens / w.mt;
        a.kgroups = w.kgroups;
        if (w.tile2d) {
            a.tile_x = w.tile_x.p;
            a.tile_y = w.tile_y.p;
        }
        // 16-byte epilogue accesses: output, residual and split-K partial rows 16-byte aligned
        // (2-D tile tables hold 64-element aligned offsets).
        const uint64_t y0 = fused ? w.y_off_run : w.y_off;
        a.epi_vec = (y0 % 8u == 0u && a.out_stride % 8u == 0u &&
                     (!w.has_res || w.res_off % 8u == 0u) &&
                     (w.kgroups <= 1u || w.part_tokens % 4u == 0u) && !w.epi_scalar)
                        ? 1u
                        : 0u;
        if (w.tile2d && w.masked) {
            a.mask_w = w.plane.W;
            a.mask_h = w.plane.H;
            a.mask_wpad = w.plane.W_pad;
            a.mask_tpf = w.tiles_per_frame;
        }
        return a;
    }

    static uint32_t epi_workgroups(const WaveExec &w) {
        if (w.kgroups <= 1u) return 0u;
        return (uint32_t)(((uint64_t)w.cout * (w.part_tokens / 4u) + 255u) / 256u);
    }

    // Device descriptors: every MFMA wave alone (command-by-command runs) and every group.
    void upload_mfma_descriptors() {
        for (auto &wp : waves) {
            WaveExec &w = *wp;
            if (!w.mfma) continue;
            w.items = w.rows * (w.narrow ? 1u : w.tokens / w.mt) * w.kgroups;
            w.epi_items = epi_workgroups(w);
            w.one_args.upload({mfma_args(w, scratch.p, false)});
            w.one_start.upload({0u, w.items});
        }
        for (auto &gp : groups) {
            MfmaGroupExec &g = *gp;
            std::vector<k44dev::MfmaTileArgs> args;
            std::vector<uint32_t> start = {0u};
            uint32_t epi_max = 0, item_max = 0;
            size_t off = 0;
            // Device order of the members: with per-wave XCD shares, waves with the most stages
            // per work item first, so that every XCD starts its longest items first.
            std::vector<size_t> order = g.members;
            if (xcd_order == 2u && g.mt != 16u)
                std::stable_sort(order.begin(), order.end(), [&](size_t p, size_t q) {
                    return item_stages(*waves[p]) > item_stages(*waves[q]);
                });
            for (size_t m : order) {
                const WaveExec &w = *waves[m];
                args.push_back(mfma_args(w, scratch.p ? scratch.p + off : nullptr, true));
                off += w.part_floats;
                start.push_back(start.back() + w.items);
                if (!w.reduce_in_kernel) epi_max = std::max(epi_max, w.epi_items);
                item_max = std::max(item_max, w.items);
            }
            g.items = start.back();
            g.epi_items = epi_max;  // epilogue grid: epi_max x members
            g.max_items = item_max;
            if (xcd_order == 2u) check_balanced_order(start);
            g.args.upload(args);
            g.start.upload(start);
        }
    }

    // Stages (k-steps for the narrow kernels) one work item of an MFMA wave runs.
    static uint32_t item_stages(const WaveExec &w) {
        const uint32_t units = w.narrow ? w.ksteps : w.K * w.S / w.rows_per_stage;
        return (units + w.kgroups - 1u) / w.kgroups;
    }

    // The per-wave XCD shares must be a bijection of the group's items (every item run by
    // exactly one workgroup); checked on the host for every group before its first launch.
    static void check_balanced_order(const std::vector<uint32_t> &start) {
        const uint32_t n = start.back(), nw = (uint32_t)start.size() - 1u;
        std::vector<uint8_t> seen(n, 0u);
        for (uint32_t b = 0; b < n; ++b) {
            uint32_t w = 0;
            const uint32_t it = k44dev::balanced_item(b, start.data(), nw, w);
            if (it >= n || seen[it] || it < start[w] || it >= start[w + 1u])
                throw std::logic_error("per-wave XCD shares are not a bijection of the items");
            seen[it] = 1u;
        }
    }

    size_t launches_per_run() const {
        size_t n = 0;
        for (const auto &r : runs) {
            if (r.first == 2) n += groups[r.second]->epi_items ? 2u : 1u;
            else if (r.first == 0 && aux[r.second]->type == K44CmdType::ARGMAX_1D)
                n += hist_steps ? 3u : 2u;
            else n += 1u;
        }
        return n;
    }

    void build_report() {
        std::ostringstream o;
        o << "{\"waves\": [";
        for (size_t i = 0; i < waves.size(); ++i) {
            const WaveExec &w = *waves[i];
            o << (i ? ", " : "") << "{\"name\": \"" << w.name << "\", \"path\": \"" << w.path
              << "\", \"why\": \"" << w.why << "\", \"cout\": " << w.cout << ", \"K\": " << w.K
              << ", \"S\": " << w.S << ", \"cluster\": " << w.cluster << ", \"step\": " << w.step
              << ", \"tokens\": " << w.tokens << ", \"slab\": " << (w.mfma ? w.mt : w.slab)
              << ", \"U\": " << (w.mfma ? w.rows_per_stage : w.U)
              << ", \"ksplit\": " << (w.mfma ? w.kgroups : w.ksplit)
              << ", \"sorted_segments\": " << (w.sorted_segments ? "true" : "false")
              << ", \"misaligned\": " << (w.misaligned ? "true" : "false")
              << ", \"phase_order\": " << (w.phase_order ? "true" : "false")
              << ", \"tokens_per_lane\": " << (w.mfma ? 0 : (w.lane8 ? 8 : 4))
              << ", \"stream_loads\": " << (w.stream_loads ? "true" : "false")
              << ", \"stream_kernel\": " << (w.stream_kernel ? "true" : "false")
              << ", \"ring_stages\": " << (w.dma ? w.dshape.nbuf : 0u)
              << ", \"ring_producers\": " << (w.dma ? w.dshape.prod : 0u)
              << ", \"xprod\": " << w.xprod
              << ", \"reduce_in_kernel\": " << (w.reduce_in_kernel ? "true" : "false")
              << ", \"flops\": " << (long long)w.flops
              << ", \"effective_flops\": " << (long long)w.eff_flops
              << ", \"mapped\": " << (w.cmap.p ? "true" : "false")
              << ", \"unique_rows\": " << w.unique_rows
              << ", \"y_off\": " << w.y_off << ", \"y_off_run\": " << w.y_off_run
              << ", \"xd\": [" << w.xd[0] << ", " << w.xd[1] << ", " << w.xd[2] << "]"
              << ", \"cmd\": " << wave_cmd[i] << "}";
        }
        o << "], \"aux\": [";
        for (size_t i = 0; i < aux.size(); ++i)
            o << (i ? ", " : "") << "{\"name\": \"" << aux[i]->name << "\", \"cmd\": " << aux_cmd[i]
              << ", \"type\": \""
              << cmd_type_str(aux[i]->type) << "\", \"channels\": " << aux[i]->D
              << ", \"fused\": " << (aux[i]->fused ? "true" : "false")
              << ", \"fuse_note\": \"" << aux[i]->fuse_note << "\""
              << ", \"chain\": " << (aux[i]->chain_inner != SIZE_MAX ? "true" : "false")
              << ", \"operands\": ["
              << (aux[i]->chain_inner != SIZE_MAX ? aux[i]->chain_other : aux[i]->src_off) << ", "
              << (aux[i]->chain_inner != SIZE_MAX ? aux[aux[i]->chain_inner]->src_off : aux[i]->src2_off)
              << ", "
              << (aux[i]->chain_inner != SIZE_MAX ? aux[aux[i]->chain_inner]->src2_off : 0u) << "]"
              << ", \"tokens\": " << aux[i]->tokens << "}";
        o << "], \"groups\": [";
        for (size_t i = 0; i < groups.size(); ++i) {
            o << (i ? ", " : "") << "[";
            for (size_t k = 0; k < groups[i]->members.size(); ++k)
                o << (k ? ", " : "") << groups[i]->members[k];
            o << "]";
        }
        // Runs of the whole-plan schedule as plan command indices (wavec_gpu_execute_runs).
        o << "], \"runs\": [";
        for (size_t r = 0; r < runs.size(); ++r) {
            std::vector<size_t> cmds;
            if (runs[r].first == 0) {
                cmds.push_back(aux_cmd[runs[r].second]);
                const size_t sw = aux[runs[r].second]->shift_with;
                if (sw != SIZE_MAX) cmds.push_back(aux_cmd[sw]);
            } else if (runs[r].first == 1) {
                cmds.push_back(wave_cmd[runs[r].second]);
            } else {
                for (size_t m : groups[runs[r].second]->members) cmds.push_back(wave_cmd[m]);
            }
            o << (r ? ", " : "") << "[";
            for (size_t k = 0; k < cmds.size(); ++k) o << (k ? ", " : "") << cmds[k];
            o << "]";
        }
        o << "], \"launches_per_run\": " << (prog_active ? (size_t)1u : launches_per_run());
        o << ", \"program\": {\"active\": " << (prog_active ? "true" : "false")
          << ", \"why\": \"" << prog_why << "\", \"stages\": " << prog_stages_h.size()
          << ", \"grid\": " << prog_grid << ", \"items\": "
          << (prog_stages_h.empty() ? 0u : prog_stages_h.back().base + prog_stages_h.back().items)
          << ", \"stage_items\": [";
        for (size_t i = 0; i < prog_stages_h.size(); ++i)
            o << (i ? ", " : "") << "[" << prog_stages_h[i].type << ", " << prog_stages_h[i].items
              << "]";
        o << "]}";
        o << ", \"canvas_elems\": " << plan_meta.canvas_elems << ", \"id_tokens\": " << id_tokens
          << "}";
        report_json = o.str();
    }

    void launch_mfma_group(const k44dev::MfmaGroup &d, uint32_t nt, uint32_t mt, uint32_t rows,
                           uint32_t items, uint32_t epi_items, bool dma, const k44dev::DmaShape &ds,
                           uint32_t prod, uint32_t max_items, bool mis) {
        if (mt == 16u)  // narrow (<= 16 tokens)
            K44_HIP(k44dev::launch_mfma_narrow(d, nt, items, stream, prod, max_items));
        else if (dma)
            K44_HIP(k44dev::launch_mfma_dma(d, nt, items, stream, ds));
        else
            K44_HIP(k44dev::launch_mfma_tile(d, nt, mt, rows, items, stream, mis));
        if (epi_items) K44_HIP(k44dev::launch_splitk_epilogue(d, epi_items, stream));
    }

    void launch_mfma(const WaveExec &w) {
        const k44dev::MfmaGroup d{w.one_args.p, w.one_start.p, 1u, xcd_order};
        launch_mfma_group(d, w.cluster, w.mt, w.rows_per_stage, w.items, w.epi_items, w.dma,
                          w.dshape, 0u, w.items, w.mis);
    }

    void launch_group(const MfmaGroupExec &g) {
        const k44dev::MfmaGroup d{g.args.p, g.start.p, (uint32_t)g.members.size(), xcd_order};
        launch_mfma_group(d, g.nt, g.mt, g.rows, g.items, g.epi_items, g.dma, g.dshape,
                          g.prod, g.max_items, g.mis);
    }

    void launch_wave(const WaveExec &w) {
        if (w.mfma) {
            launch_mfma(w);
            if (w.tile2d)
                K44_HIP(k44dev::launch_halo_clear(canvas.p + w.y_off, w.cout, w.plane, stream));
            return;
        }
        if (w.tile2d) {
            k44dev::GatherTileArgs a{};
            a.X = canvas.p;
            a.seg = w.seg.p;
            a.W = w.w.p;
            a.bias = w.bias.p;
            a.cmap = w.cmap.p;
            a.Y = canvas.p + w.y_off;
            a.R = w.has_res ? canvas.p + w.res_off : nullptr;
            a.tile_x = w.tile_x.p;
            a.tile_y = w.tile_y.p;
            a.step = w.step;
            a.K = w.K;
            a.S = w.S;
            a.cluster = w.cluster;
            a.cout = w.cout;
            a.tiles = w.tiles;
            a.out_stride = w.plane.channel_stride;
            a.act = w.act;
            a.plane = w.plane;
            a.tiles_per_frame = w.tiles_per_frame;
            a.masked = w.masked;
            K44_HIP(k44dev::launch_gather_tile(a, stream));
            K44_HIP(k44dev::launch_halo_clear(canvas.p + w.y_off, w.cout, w.plane, stream));
            return;
        }
        k44dev::GatherDotArgs a{};
        a.X = canvas.p;
        a.seg = w.seg.p;
        a.W = w.w.p;
        a.bias = w.bias.p;
        a.cmap = w.cmap.p;
        a.Y = canvas.p + w.y_off;
        a.R = w.has_res ? canvas.p + w.res_off : nullptr;
        a.step = w.step;
        a.K = w.K;
        a.S = w.S;
        a.n_batch = w.n_batch;
        a.cluster = w.cluster;
        a.cout = w.cout;
        a.out_stride = w.out_stride;
        a.act = w.act;
        if (w.stream_kernel)
            K44_HIP(k44dev::launch_gather_stream(a, w.tokens, stream, w.stream_loads));
        else
            K44_HIP(k44dev::launch_gather_dot(a, w.slab, w.ksplit, w.tokens, stream, w.lane8,
                                              w.stream_loads, w.weights_in_lds, w.misaligned));
    }

    void launch_op(size_t i) {
        const auto &op = ops.at(i);
        if (op.first)
            launch_wave(*waves[op.second]);
        else
            launch_aux(*aux[op.second]);
    }

    void launch_ops(size_t first = 0, size_t n = SIZE_MAX) {
        const size_t end = n == SIZE_MAX ? runs.size() : std::min(runs.size(), first + n);
        for (size_t i = first; i < end; ++i) {
            const auto &r = runs[i];
            if (r.first == 0)
                launch_aux(*aux[r.second], true);
            else if (r.first == 1)
                launch_wave(*waves[r.second]);
            else
                launch_group(*groups[r.second]);
        }
    }

    // One plan run on the executor stream: kernel by kernel, or as one replay of a HIP graph
    // captured from the same launches (no memset/memcpy nodes in it).
    void execute_plan() {
        if (prog_active) {  // one launch: nothing to capture
            K44_HIP(k44dev::launch_program(prog_args, prog_grid, stream));
            return;
        }
        if (!use_graph) {
            launch_ops();
            return;
        }
        if (!graph_exec) {
            K44_HIP(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
            try {
                launch_ops();
            } catch (...) {
                hipGraph_t g = nullptr;
                (void)hipStreamEndCapture(stream, &g);
                if (g) (void)hipGraphDestroy(g);
                throw;
            }
            K44_HIP(hipStreamEndCapture(stream, &graph));
            K44_HIP(hipGraphInstantiate(&graph_exec, graph, nullptr, nullptr, 0));
        }
        K44_HIP(hipGraphLaunch(graph_exec, stream));
    }

    void set_history(uint32_t steps) {
        if (!id_tokens) throw std::runtime_error("plan has no token-id buffer (no embed/argmax)");
        K44_HIP(hipStreamSynchronize(stream));
        drop_graph();  // the history pointer is baked into captured launches
        history.alloc((size_t)std::max(1u, steps) * id_tokens);
        hist_steps = steps;
        K44_HIP(hipMemsetAsync(history.p, 0, history.n * 4u, stream));
        K44_HIP(hipMemsetAsync(step_ctr.p, 0, 4u, stream));
        K44_HIP(hipStreamSynchronize(stream));
        if (prog_active) build_program();  // the history pointer is in its argmax stage
    }

    const K44ResDesc &layout(uint32_t key) const { return plan_meta.res_map.at(key); }

    void upload_input_f32(const float *in, size_t n) {
        const K44ResDesc &L = layout(plan_meta.input_res_key);
        // whole planes (zero halos): the region may hold another tensor's data from the last run
        std::vector<uint16_t> pad((size_t)plan_meta.input_c * L.channel_stride, 0u);
        for (uint32_t ch = 0; ch < plan_meta.input_c; ++ch)
            for (uint32_t y = 0; y < plan_meta.input_h; ++y)
                for (uint32_t x = 0; x < plan_meta.input_w; ++x) {
                    const size_t src = ((size_t)ch * plan_meta.input_h + y) * plan_meta.input_w + x;
                    if (src < n) pad[L.canvas_offset(ch, y, x)] = float_to_half(in[src]);
                }
        K44_HIP(hipMemcpyAsync(canvas.p + plan_meta.input_off, pad.data(), pad.size() * 2u,
                               hipMemcpyHostToDevice, stream));
        K44_HIP(hipStreamSynchronize(stream));
    }

    std::vector<float> download_output_f32() {
        const K44ResDesc &L = layout(plan_meta.output_res_key);
        std::vector<uint16_t> pad((size_t)plan_meta.output_c * L.channel_stride);
        K44_HIP(hipMemcpyAsync(pad.data(), canvas.p + plan_meta.output_off, pad.size() * 2u,
                               hipMemcpyDeviceToHost, stream));
        K44_HIP(hipStreamSynchronize(stream));
        std::vector<float> out((size_t)plan_meta.output_c * plan_meta.output_h * plan_meta.output_w);
        for (uint32_t ch = 0; ch < plan_meta.output_c; ++ch)
            for (uint32_t y = 0; y < plan_meta.output_h; ++y)
                for (uint32_t x = 0; x < plan_meta.output_w; ++x)
                    out[((size_t)ch * plan_meta.output_h + y) * plan_meta.output_w + x] =
                        half_to_float(pad[L.canvas_offset(ch, y, x)]);
        return out;
    }

    int infer_f32(const float *in, int in_elems, float *out, int out_elems, float *ms_out) {
        if (!initialized) throw std::runtime_error("executor not initialised");
        upload_input_f32(in, (size_t)std::max(0, in_elems));
        K44_HIP(hipEventRecord(ev0, stream));
        execute_plan();
        K44_HIP(hipEventRecord(ev1, stream));
        K44_HIP(hipEventSynchronize(ev1));
        float ms = 0.0f;
        K44_HIP(hipEventElapsedTime(&ms, ev0, ev1));
        if (ms_out) *ms_out = ms;
        const std::vector<float> y = download_output_f32();
        std::memcpy(out, y.data(), std::min((size_t)std::max(0, out_elems), y.size()) * 4u);
        return 0;
    }
};

// Workspace of the allocation-free entry points: an array in the library's device code
// object, so each GPU the library runs on holds its own copy until the process ends.  Host code
// never passes the array's name to a kernel (on the host it is only a stand-in for the symbol):
// scratch_ptr() looks up its address on the current device once (hipGetSymbolAddress) and keeps
// it per device.  Every call on one GPU shares that GPU's copy: calls that overlap on one GPU
// (different streams, different threads) race.
namespace noalloc {
constexpr size_t kScratchFloats = (size_t)1 << 20;  // 4 MiB
static __device__ __align__(256) float scratch[kScratchFloats];
static std::mutex g_mu;
static std::map<int, float *> g_ptr;  // device ordinal -> address of `scratch` there

static float *scratch_ptr() {
    int dev = 0;
    K44_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_ptr.find(dev);
    if (it != g_ptr.end()) return it->second;
    void *p = nullptr;
    K44_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) throw std::runtime_error("hipGetSymbolAddress returned no address for the workspace");
    g_ptr[dev] = static_cast<float *>(p);
    return g_ptr[dev];
}
}  // namespace noalloc

static std::mutex g_exec_mu;
// Executors by graph handle.  Heap-held and never destroyed, so no HIP call runs from a static
// destructor after the HIP runtime has shut down at process exit.
static auto &g_gpu_executors = *new std::map<void *, std::unique_ptr<K44GpuExecutorState>>();

static K44GpuExecutorState *find_exec(void *h) {
    std::lock_guard<std::mutex> lk(g_exec_mu);
    auto it = g_gpu_executors.find(h);
    return (it == g_gpu_executors.end() || !it->second || !it->second->initialized)
               ? nullptr
               : it->second.get();
}

}  // namespace k44_host

// =================================================================================================
// C ABI
// =================================================================================================
using k44_host::K44Act;
using k44_host::K44WaveGraphCompiler;

namespace {

K44WaveGraphCompiler *comp_of(void *h) { return static_cast<K44WaveGraphCompiler *>(h); }

// Runs f, mapping every exception to -1 + last-error text.
template <typename F>
int guarded(const char *what, F &&f) {
    try {
        return f();
    } catch (const std::exception &e) {
        set_error(std::string(what) + ": " + e.what());
    } catch (...) {
        set_error(std::string(what) + ": unknown error");
    }
    (void)hipGetLastError();  // a failed runtime call must not resurface at the next launch
    return -1;
}

K44WaveGraphCompiler *compiled(void *h) {
    K44WaveGraphCompiler *c = comp_of(h);
    if (c && !c->is_compiled) c->compile();
    return c;
}

std::string opt_str(const char *s) { return s ? std::string(s) : std::string(); }

}  // namespace

extern "C" {

void *wavec_create(int max_B_per_wave, int default_S, int kv_cache_max_seq,
                   int fold_rmsnorm_gamma) {
    auto *c = new K44WaveGraphCompiler();
    c->opts.max_B_per_wave = (uint32_t)std::max(0, max_B_per_wave);
    c->opts.force_cluster_size = (uint32_t)std::max(0, default_S);
    c->opts.kv_cache_max_seq = (uint32_t)std::max(0, kv_cache_max_seq);
    c->opts.fold_rmsnorm_gamma = fold_rmsnorm_gamma != 0;
    c->opts.keep_host_plan_buffers = true;
    return c;
}

void wavec_destroy(void *h) {
    if (!h) return;
    {
        std::lock_guard<std::mutex> lk(k44_host::g_exec_mu);
        k44_host::g_gpu_executors.erase(h);
    }
    delete comp_of(h);
}

int wavec_gpu_release(void *h) {
    if (!h) return -1;
    std::lock_guard<std::mutex> lk(k44_host::g_exec_mu);
    k44_host::g_gpu_executors.erase(h);
    return 0;
}

int wavec_add_input(void *h, const char *name, int c, int hh, int w, int is_1d) {
    if (!h || !name) return -1;
    return guarded("wavec_add_input", [&] {
        comp_of(h)->add_input(name, (uint32_t)c, (uint32_t)hh, (uint32_t)w, is_1d != 0);
        return 0;
    });
}

int wavec_add_flatten(void *h, const char *name, const char *in, const char *out) {
    if (!h || !name || !in || !out) return -1;
    return guarded("wavec_add_flatten", [&] {
        comp_of(h)->add_flatten(name, in, out);
        return 0;
    });
}

int wavec_add_conv2d(void *h, const char *name, const char *in, const char *out, int cin,
                     int cout, int kh, int kw, int stride, int pad, int act, const float *w_f32,
                     const float *bias_f32, const char *residual) {
    if (!h || !name || !in || !out) return -1;
    return guarded("wavec_add_conv2d", [&] {
        comp_of(h)->add_conv2d(name, in, out, (uint32_t)cin, (uint32_t)cout, (uint32_t)kh,
                               (uint32_t)kw, (uint32_t)stride, (uint32_t)pad, (K44Act)act, w_f32,
                               bias_f32, opt_str(residual));
        return 0;
    });
}

int wavec_add_conv2d_f16(void *h, const char *name, const char *in, const char *out, int cin,
                         int cout, int kh, int kw, int stride, int pad, int act,
                         const uint16_t *w_f16, const float *bias_f32, const char *residual) {
    if (!h || !name || !in || !out) return -1;
    return guarded("wavec_add_conv2d_f16", [&] {
        comp_of(h)->add_conv2d_f16(name, in, out, (uint32_t)cin, (uint32_t)cout, (uint32_t)kh,
                                   (uint32_t)kw, (uint32_t)stride, (uint32_t)pad, (K44Act)act,
                                   w_f16, bias_f32, opt_str(residual));
        return 0;
    });
}

int wavec_add_linear_f32(void *h, const char *name, const char *in, const char *out, int din,
                         int dout, int act, const float *w_f32, const float *bias_f32,
                         const char *residual) {
    return wavec_add_conv2d(h, name, in, out, din, dout, 1, 1, 1, 0, act, w_f32, bias_f32,
                            residual);
}

int wavec_add_linear_f16(void *h, const char *name, const char *in, const char *out, int din,
                         int dout, int act, const uint16_t *w_f16, const float *bias_f32,
                         const char *residual) {
    return wavec_add_conv2d_f16(h, name, in, out, din, dout, 1, 1, 1, 0, act, w_f16, bias_f32,
                                residual);
}

int wavec_add_linear_bf16(void *h, const char *name, const char *in, const char *out, int din,
                          int dout, int act, const uint16_t *w_bf16, const float *bias_f32,
                          const char *residual) {
    if (!h || !name || !in || !out) return -1;
    return guarded("wavec_add_linear_bf16", [&] {
        comp_of(h)->add_linear_bf16(name, in, out, (uint32_t)din, (uint32_t)dout, (K44Act)act,
                                    w_bf16, bias_f32, opt_str(residual));
        return 0;
    });
}

int wavec_add_upconv2x2(void *h, const char *name, const char *in, const char *out, int cin,
                        int cout, const float *w_f32, const float *bias_f32) {
    if (!h || !name || !in || !out) return -1;
    return guarded("wavec_add_upconv2x2", [&] {
        comp_of(h)->add_upconv2x2(name, in, out, (uint32_t)cin, (uint32_t)cout, w_f32, bias_f32);
        return 0;
    });
}

int wavec_add_maxpool(void *h, const char *name, const char *in, const char *out, int k,
                      int stride, int pad) {
    if (!h || !name || !in || !out) return -1;
    return guarded("wavec_add_maxpool", [&] {
        comp_of(h)->add_maxpool(name, in, out, (uint32_t)k, (uint32_t)stride, (uint32_t)pad);
        return 0;
    });
}

int wavec_add_upsample2x(void *h, const char *name, const char *in, const char *out) {
    if (!h || !name || !in || !out) return -1;
    return guarded("wavec_add_upsample2x", [&] {
        comp_of(h)->add_upsample2x(name, in, out);
        return 0;
    });
}

int wavec_add_rmsnorm(void *h, const char *name, const char *in, const char *out, int dim,
                      float eps, const float *gamma_f32, int pre_folded) {
    if (!h || !name || !in || !out) return -1;
    return guarded("wavec_add_rmsnorm", [&] {
        comp_of(h)->add_rmsnorm(name, in, out, (uint32_t)dim, eps, gamma_f32, pre_folded != 0);
        return 0;
    });
}

int wavec_add_swiglu(void *h, const char *name, const char *gate, const char *up,
                     const char *out) {
    if (!h || !name || !gate || !up || !out) return -1;
    return guarded("wavec_add_swiglu", [&] {
        comp_of(h)->add_swiglu_mul(name, gate, up, out);
        return 0;
    });
}

int wavec_add_rope_gqa_attn(void *h, const char *name, const char *q, const char *k,
                            const char *v, const char *out, int h_q, int h_kv, int head_dim,
                            float rope_theta, int llama3_scaling) {
    if (!h || !name || !q || !k || !v || !out) return -1;
    return guarded("wavec_add_rope_gqa_attn", [&] {
        comp_of(h)->add_rope_gqa_attention(name, q, k, v, out, (uint32_t)h_q, (uint32_t)h_kv,
                                           (uint32_t)head_dim, rope_theta, llama3_scaling != 0);
        return 0;
    });
}

int wavec_add_split(void *h, const char *name, const char *in, int num_outs, const char **outs) {
    if (!h || !name || !in || num_outs <= 0 || !outs) return -1;
    return guarded("wavec_add_split", [&] {
        comp_of(h)->add_split(name, in, std::vector<std::string>(outs, outs + num_outs));
        return 0;
    });
}

int wavec_add_slice(void *h, const char *name, const char *in, int num_outs, const char **outs,
                    const int *slice_sizes) {
    if (!h || !name || !in || num_outs <= 0 || !outs) return -1;
    return guarded("wavec_add_slice", [&] {
        std::vector<uint32_t> sizes;
        if (slice_sizes)
            for (int i = 0; i < num_outs; ++i) sizes.push_back((uint32_t)slice_sizes[i]);
        comp_of(h)->add_slice(name, in, std::vector<std::string>(outs, outs + num_outs), sizes);
        return 0;
    });
}

int wavec_add_concat(void *h, const char *name, int num_ins, const char **ins, const char *out) {
    if (!h || !name || num_ins <= 0 || !ins || !out) return -1;
    return guarded("wavec_add_concat", [&] {
        comp_of(h)->add_concat(name, std::vector<std::string>(ins, ins + num_ins), out);
        return 0;
    });
}

int wavec_set_output(void *h, const char *out) {
    if (!h || !out) return -1;
    comp_of(h)->default_output_tensor = out;
    comp_of(h)->is_compiled = false;
    return 0;
}

int wavec_set_reuse_canvas(void *h, int reuse) {
    if (!h) return -1;
    comp_of(h)->opts.reuse_canvas = reuse != 0;
    comp_of(h)->is_compiled = false;
    return 0;
}

int wavec_set_batch_size(void *h, int batch) {
    if (!h) return -1;
    comp_of(h)->opts.batch_size = (uint32_t)std::max(1, batch);
    comp_of(h)->is_compiled = false;
    return 0;
}

int wavec_set_target_preset(void *h, const char *preset) {
    if (!h) return -1;
    comp_of(h)->opts.hw_profile = k44_host::K44HardwareProfile::from_preset(preset);
    comp_of(h)->is_compiled = false;
    return 0;
}

int wavec_compile(void *h) {
    if (!h) return -1;
    return guarded("wavec_compile", [&] {
        comp_of(h)->compile();
        return 0;
    });
}

const char *wavec_get_summary_json(void *h) {
    if (!h) return "{}";
    if (guarded("wavec_get_summary_json", [&] {
            compiled(h);
            return 0;
        }) != 0)
        return "{}";
    return comp_of(h)->cached_summary_json.c_str();
}

int wavec_save_tcff_ex(void *h, const char *path, const char *prefix, int include_canvas,
                       int include_geometry) {
    if (!h || !path) return -1;
    (void)include_canvas;  // as in the reference: canvas pages are never written
    return guarded("wavec_save_tcff", [&] {
        return k44_host::save_plan_to_tcff(compiled(h)->compiled_plan, path, prefix, false,
                                           include_geometry != 0, nullptr)
                   ? 0
                   : -1;
    });
}

int wavec_save_tcff(void *h, const char *path, const char *prefix) {
    return wavec_save_tcff_ex(h, path, prefix, 1, 1);
}

int wavec_load_tcff_weights(void *h, const char *path) {
    if (!h || !path) return -1;
    return guarded("wavec_load_tcff_weights", [&] {
        if (!k44_host::load_weights_from_tcff(compiled(h)->compiled_plan, path)) {
            set_error(std::string("wavec_load_tcff_weights: rejected ") + path);
            return -1;
        }
        return 0;
    });
}

int wavec_gpu_init_plan(void *h) {
    if (!h) return -1;
    return guarded("wavec_gpu_init_plan", [&] {
        K44WaveGraphCompiler *c = compiled(h);
        auto ex = std::make_unique<k44_host::K44GpuExecutorState>();
        ex->init(c->compiled_plan);
        std::lock_guard<std::mutex> lk(k44_host::g_exec_mu);
        k44_host::g_gpu_executors[h] = std::move(ex);
        return 0;
    });
}

int wavec_gpu_infer_f32(void *h, const float *in, int in_elems, float *out, int out_elems,
                        float *out_gpu_ms) {
    if (!h || !in || !out) return -1;
    return guarded("wavec_gpu_infer_f32", [&] {
        k44_host::K44GpuExecutorState *ex = k44_host::find_exec(h);
        if (!ex) throw std::runtime_error("wavec_gpu_init_plan has not succeeded for this handle");
        return ex->infer_f32(in, in_elems, out, out_elems, out_gpu_ms);
    });
}

// ------------------------------- build extensions --------------------------------------------

const char *wavec_last_error(void) { return g_last_error.c_str(); }

int wavec_add_sparse_wave(void *h, const char *name, const char *in, const char *out, int cout,
                          int fan_in, int cluster, const uint32_t *rows, const uint16_t *w_f16,
                          const uint16_t *bias_f16, int act, const char *residual) {
    if (!h || !name || !in || !out || cout <= 0 || fan_in <= 0 || cluster <= 0) return -1;
    return guarded("wavec_add_sparse_wave", [&] {
        comp_of(h)->add_sparse_wave(name, in, out, (uint32_t)cout, (uint32_t)fan_in,
                                    (uint32_t)cluster, rows, w_f16, bias_f16, (K44Act)act,
                                    opt_str(residual));
        return 0;
    });
}

int wavec_add_cluster_wave(void *h, const char *name, const char *in, const char *out, int cout,
                           int K, int S, int cluster, const uint32_t *starts,
                           const uint16_t *w_f16, const uint16_t *bias_f16, int act,
                           const char *residual) {
    if (!h || !name || !in || !out || cout <= 0 || K <= 0 || S <= 0 || cluster <= 0) return -1;
    return guarded("wavec_add_cluster_wave", [&] {
        comp_of(h)->add_cluster_wave(name, in, out, (uint32_t)cout, (uint32_t)K, (uint32_t)S,
                                     (uint32_t)cluster, starts, w_f16, bias_f16, (K44Act)act,
                                     opt_str(residual));
        return 0;
    });
}

int wavec_add_pruned_wave(void *h, const char *name, const char *in, const char *out, int cout,
                          int K, int S, int tile, const uint32_t *starts, const uint16_t *w_f16,
                          const uint16_t *bias_f16, int act, const char *residual) {
    if (!h || !name || !in || !out || cout <= 0 || K <= 0 || S <= 0 || tile <= 0) return -1;
    return guarded("wavec_add_pruned_wave", [&] {
        comp_of(h)->add_pruned_wave(name, in, out, (uint32_t)cout, (uint32_t)K, (uint32_t)S,
                                    (uint32_t)tile, starts, w_f16, bias_f16, (K44Act)act,
                                    opt_str(residual));
        return 0;
    });
}

int wavec_gpu_fill_input_uniform(void *h, unsigned long long seed) {
    if (!h) return -1;
    return guarded("wavec_gpu_fill_input_uniform", [&] {
        k44_host::K44GpuExecutorState *ex = k44_host::find_exec(h);
        if (!ex) throw std::runtime_error("wavec_gpu_init_plan has not succeeded for this handle");
        const auto &L = ex->layout(ex->plan_meta.input_res_key);
        if (!L.is_1d_tokens) throw std::runtime_error("2-D input layouts are not supported");
        const uint64_t rows = ex->plan_meta.input_c;
        K44_HIP(k44dev::launch_fill_uniform(ex->canvas.p + ex->plan_meta.input_off, rows,
                                            L.channel_stride, ex->plan_meta.input_w, 0u,
                                            (uint64_t)seed, ex->stream));
        K44_HIP(hipStreamSynchronize(ex->stream));
        return 0;
    });
}

void *wavec_dev_malloc(unsigned long long bytes) {
    void *p = nullptr;
    const int rc = guarded("wavec_dev_malloc", [&] {
        K44_HIP(hipMalloc(&p, bytes ? bytes : 1u));
        return 0;
    });
    return rc == 0 ? p : nullptr;
}

int wavec_dev_free(void *p) {
    return guarded("wavec_dev_free", [&] {
        if (p) K44_HIP(hipFree(p));
        return 0;
    });
}

int wavec_dev_upload(void *dst, const void *src, unsigned long long bytes) {
    if (!dst || !src) return -1;
    return guarded("wavec_dev_upload", [&] {
        K44_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
        return 0;
    });
}

int wavec_dev_download(void *dst, const void *src, unsigned long long bytes) {
    if (!dst || !src) return -1;
    return guarded("wavec_dev_download", [&] {
        K44_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
        return 0;
    });
}

int wavec_dev_synchronize(void) {
    return guarded("wavec_dev_synchronize", [&] {
        K44_HIP(hipDeviceSynchronize());
        return 0;
    });
}

int wavec_dev_fill_uniform(void *dst, unsigned long long rows, unsigned int stride,
                           unsigned int valid, unsigned long long pos0, unsigned long long seed) {
    if (!dst || stride == 0u || valid > stride) return -1;
    return guarded("wavec_dev_fill_uniform", [&] {
        K44_HIP(k44dev::launch_fill_uniform(static_cast<__half *>(dst), rows, stride, valid, pos0,
                                            seed, nullptr));
        K44_HIP(hipDeviceSynchronize());
        return 0;
    });
}

namespace {
hipEvent_t g_t0 = nullptr, g_t1 = nullptr;  // null-stream timer of the stand-alone kernels
}

int wavec_dev_time_begin(void) {
    return guarded("wavec_dev_time_begin", [&] {
        if (!g_t0) K44_HIP(hipEventCreate(&g_t0));
        if (!g_t1) K44_HIP(hipEventCreate(&g_t1));
        K44_HIP(hipEventRecord(g_t0, nullptr));
        return 0;
    });
}

int wavec_dev_time_end(float *ms) {
    if (!ms) return -1;
    return guarded("wavec_dev_time_end", [&] {
        if (!g_t0 || !g_t1) throw std::runtime_error("wavec_dev_time_begin was not called");
        K44_HIP(hipEventRecord(g_t1, nullptr));
        K44_HIP(hipEventSynchronize(g_t1));
        K44_HIP(hipEventElapsedTime(ms, g_t0, g_t1));
        return 0;
    });
}

int wavec_k44_f16_forward_token64(void *Y, const void *X, const uint32_t *cluster_indices,
                                  const void *cluster_weights_wmma, const void *neuron_bias,
                                  uint32_t batch_size, uint32_t Cin, uint32_t Cout,
                                  uint32_t B_vec16, uint32_t cluster_size, void *stream) {
    return guarded("wavec_k44_f16_forward_token64", [&] {
        if (!Y || !X || !cluster_indices || !cluster_weights_wmma)
            throw std::runtime_error("Y, X, cluster_indices and cluster_weights_wmma are required");
        if (batch_size == 0u || Cin == 0u || B_vec16 == 0u)
            throw std::runtime_error("batch_size, Cin and B_vec16 must be positive");
        if (cluster_size < 16u || cluster_size % 16u != 0u || Cout == 0u || Cout % cluster_size != 0u)
            throw std::runtime_error("cluster_size must be a multiple of 16 that divides Cout");
        const uint32_t tiles = (batch_size + 63u) / 64u;
        if ((tiles + 3u) / 4u > 65535u) throw std::runtime_error("batch_size too large");
        k44dev::Token64Args a{};
        a.Y = static_cast<__half *>(Y);
        a.X = static_cast<const __half *>(X);
        a.idx = cluster_indices;
        a.w_wmma = static_cast<const uint4 *>(cluster_weights_wmma);
        a.bias = static_cast<const __half *>(neuron_bias);
        a.Cin = Cin;
        a.Cout = Cout;
        a.B_vec16 = B_vec16;
        a.cluster = cluster_size;
        a.tiles = tiles;
        K44_HIP(k44dev::launch_token64(a, static_cast<hipStream_t>(stream),
                                       k44_host::tune(k44_host::Tune::Token64Ring)));
        return 0;
    });
}

// The argmax kernels read logits with 8- or 16-byte loads (16 when the pointer allows) and
// store 4-byte ids: a pointer off those boundaries is refused before anything is launched.
static void check_argmax_alignment(const uint32_t *ids, const void *logits) {
    if (reinterpret_cast<uintptr_t>(logits) % 8u != 0u)
        throw std::runtime_error("logits must be 8-byte aligned (a multiple of 4 fp16 elements)");
    if (reinterpret_cast<uintptr_t>(ids) % 4u != 0u)
        throw std::runtime_error("ids must be 4-byte aligned");
}

int wavec_argmax_f16(uint32_t *ids, const void *logits, uint32_t vocab, uint32_t stride,
                     uint32_t tokens, void *stream) {
    return guarded("wavec_argmax_f16", [&] {
        if (!ids || !logits) throw std::runtime_error("ids and logits are required");
        check_argmax_alignment(ids, logits);
        if (vocab == 0u || stride == 0u || stride % 64u != 0u || tokens == 0u || tokens > stride)
            throw std::runtime_error("vocab > 0, stride a positive multiple of 64 and "
                                     "0 < tokens <= stride are required");
        const hipStream_t st = static_cast<hipStream_t>(stream);
        // Per-chunk (value, index) partials: a stream-ordered workspace for this call.
        const size_t bytes = k44dev::argmax_scratch_floats(vocab, stride) * sizeof(float);
        void *work = nullptr;
        K44_HIP(hipMallocAsync(&work, bytes, st));
        const hipError_t e = k44dev::launch_argmax(ids, nullptr, nullptr, 0u,
                                                   static_cast<const __half *>(logits), vocab,
                                                   stride, tokens, static_cast<float *>(work), st);
        K44_HIP(hipFreeAsync(work, st));
        K44_HIP(e);
        return 0;
    });
}

int wavec_argmax_f16_noalloc(uint32_t *ids, const void *logits, uint32_t vocab,
                             uint32_t stride, uint32_t tokens, void *stream) {
    return guarded("wavec_argmax_f16_noalloc", [&] {
        if (!ids || !logits) throw std::runtime_error("ids and logits are required");
        check_argmax_alignment(ids, logits);
        if (vocab == 0u || stride == 0u || stride % 64u != 0u || tokens == 0u || tokens > stride)
            throw std::runtime_error("vocab > 0, stride a positive multiple of 64 and "
                                     "0 < tokens <= stride are required");
        const size_t need = k44dev::argmax_scratch_floats(vocab, stride);
        if (need > k44_host::noalloc::kScratchFloats)
            throw std::runtime_error("needs " + std::to_string(need) +
                                     " floats of workspace; the allocation-free form holds " +
                                     std::to_string(k44_host::noalloc::kScratchFloats) +
                                     " (use wavec_argmax_f16 for this size)");
        float *ws = k44_host::noalloc::scratch_ptr();
        K44_HIP(k44dev::launch_argmax(ids, nullptr, nullptr, 0u,
                                      static_cast<const __half *>(logits), vocab, stride, tokens,
                                      ws, static_cast<hipStream_t>(stream)));
        return 0;
    });
}

int wavec_interleave_weights_wmma(void *dst_wmma, const void *src_compact,
                                  uint32_t num_output_neurons, uint32_t B_vec8, void *stream) {
    return guarded("wavec_interleave_weights_wmma", [&] {
        if (!dst_wmma || !src_compact) throw std::runtime_error("null device pointer");
        if (num_output_neurons % 16u != 0u || B_vec8 == 0u || B_vec8 % 2u != 0u)
            throw std::runtime_error("num_output_neurons must be a multiple of 16 and B_vec8 even");
        K44_HIP(k44dev::launch_interleave_wmma(static_cast<uint4 *>(dst_wmma),
                                               static_cast<const uint4 *>(src_compact),
                                               num_output_neurons, B_vec8,
                                               static_cast<hipStream_t>(stream)));
        return 0;
    });
}

int wavec_gpu_execute(void *h, int iters, float *out_ms_per_iter) {
    if (!h || iters <= 0) return -1;
    return guarded("wavec_gpu_execute", [&] {
        k44_host::K44GpuExecutorState *ex = k44_host::find_exec(h);
        if (!ex) throw std::runtime_error("wavec_gpu_init_plan has not succeeded for this handle");
        K44_HIP(hipEventRecord(ex->ev0, ex->stream));
        for (int i = 0; i < iters; ++i) ex->execute_plan();
        K44_HIP(hipEventRecord(ex->ev1, ex->stream));
        K44_HIP(hipEventSynchronize(ex->ev1));
        ex->check_program();
        float ms = 0.0f;
        K44_HIP(hipEventElapsedTime(&ms, ex->ev0, ex->ev1));
        if (out_ms_per_iter) *out_ms_per_iter = ms / (float)iters;
        return 0;
    });
}

int wavec_gpu_execute_range(void *h, int first_cmd, int n_cmds) {
    if (!h || first_cmd < 0 || n_cmds < 0) return -1;
    return guarded("wavec_gpu_execute_range", [&] {
        k44_host::K44GpuExecutorState *ex = k44_host::find_exec(h);
        if (!ex) throw std::runtime_error("wavec_gpu_init_plan has not succeeded for this handle");
        if ((size_t)first_cmd + (size_t)n_cmds > ex->ops.size())
            throw std::runtime_error("command range past the end of the plan");
        for (int i = first_cmd; i < first_cmd + n_cmds; ++i) ex->launch_op((size_t)i);
        K44_HIP(hipStreamSynchronize(ex->stream));
        return 0;
    });
}

int wavec_gpu_program_trace(void *h, unsigned long long *dst, unsigned long long n_words) {
    if (!h || !dst) return -1;
    return guarded("wavec_gpu_program_trace", [&] {
        k44_host::K44GpuExecutorState *ex = k44_host::find_exec(h);
        if (!ex) throw std::runtime_error("wavec_gpu_init_plan has not succeeded for this handle");
        if (!ex->prog_trace.p)
            throw std::runtime_error("no program trace (a persistent launch built with prog_trace=1)");
        if (n_words > ex->prog_trace.n) throw std::runtime_error("more words than the trace holds");
        K44_HIP(hipMemcpyAsync(dst, ex->prog_trace.p, n_words * 8u, hipMemcpyDeviceToHost,
                               ex->stream));
        K44_HIP(hipStreamSynchronize(ex->stream));
        return 0;
    });
}

int wavec_gpu_sync(void *h) {
    if (!h) return -1;
    return guarded("wavec_gpu_sync", [&] {
        k44_host::K44GpuExecutorState *ex = k44_host::find_exec(h);
        if (!ex) throw std::runtime_error("wavec_gpu_init_plan has not succeeded for this handle");
        K44_HIP(hipStreamSynchronize(ex->stream));
        ex->check_program();
        return 0;
    });
}

int wavec_gpu_read_canvas(void *h, unsigned long long off, unsigned long long n, uint16_t *dst) {
    if (!h || (!dst && n)) return -1;
    return guarded("wavec_gpu_read_canvas", [&] {
        k44_host::K44GpuExecutorState *ex = k44_host::find_exec(h);
        if (!ex) throw std::runtime_error("wavec_gpu_init_plan has not succeeded for this handle");
        if (off > ex->plan_meta.canvas_elems || n > ex->plan_meta.canvas_elems - off)
            throw std::runtime_error("range outside the canvas");
        K44_HIP(hipMemcpyAsync(dst, ex->canvas.p + off, n * 2u, hipMemcpyDeviceToHost, ex->stream));
        K44_HIP(hipStreamSynchronize(ex->stream));
        return 0;
    });
}

int wavec_gpu_write_canvas(void *h, unsigned long long off, unsigned long long n,
                           const uint16_t *src) {
    if (!h || (!src && n)) return -1;
    return guarded("wavec_gpu_write_canvas", [&] {
        k44_host::K44GpuExecutorState *ex = k44_host::find_exec(h);
        if (!ex) throw std::runtime_error("wavec_gpu_init_plan has not succeeded for this handle");
        if (off > ex->plan_meta.canvas_elems || n > ex->plan_meta.canvas_elems - off)
            throw std::runtime_error("range outside the canvas");
        K44_HIP(hipMemcpyAsync(ex->canvas.p + off, src, n * 2u, hipMemcpyHostToDevice, ex->stream));
        K44_HIP(hipStreamSynchronize(ex->stream));
        return 0;
    });
}

int wavec_add_token_shift(void *h, const char *name, const char *in, const char *out, int dim,
                          int rf, int seq_len, const uint16_t *mu_f16, int decode) {
    if (!h || !name || !in || !out || dim <= 0 || rf <= 0 || seq_len <= 0) return -1;
    return guarded("wavec_add_token_shift", [&] {
        comp_of(h)->add_token_shift(name, in, out, (uint32_t)dim, (uint32_t)rf,
                                    (uint32_t)seq_len, mu_f16, decode != 0);
        return 0;
    });
}

int wavec_add_embedding(void *h, const char *name, const char *tok_in, const char *out,
                        int vocab, int dim, const uint16_t *table_f16) {
    if (!h || !name || !tok_in || !out || vocab <= 0 || dim <= 0) return -1;
    return guarded("wavec_add_embedding", [&] {
        comp_of(h)->add_embedding(name, tok_in, out, (uint32_t)vocab, (uint32_t)dim, table_f16);
        return 0;
    });
}

int wavec_add_argmax(void *h, const char *name, const char *in, const char *out) {
    if (!h || !name || !in || !out) return -1;
    return guarded("wavec_add_argmax", [&] {
        comp_of(h)->add_argmax(name, in, out);
        return 0;
    });
}

static k44_host::K44GpuExecutorState *exec_or_throw(void *h) {
    k44_host::K44GpuExecutorState *ex = k44_host::find_exec(h);
    if (!ex) throw std::runtime_error("wavec_gpu_init_plan has not succeeded for this handle");
    return ex;
}

int wavec_gpu_set_ids(void *h, const uint32_t *ids, int n) {
    if (!h || !ids || n < 0) return -1;
    return guarded("wavec_gpu_set_ids", [&] {
        auto *ex = exec_or_throw(h);
        if ((uint32_t)n > ex->id_tokens) throw std::runtime_error("more ids than plan tokens");
        K44_HIP(hipMemcpyAsync(ex->ids.p, ids, (size_t)n * 4u, hipMemcpyHostToDevice, ex->stream));
        K44_HIP(hipStreamSynchronize(ex->stream));
        return 0;
    });
}

int wavec_gpu_get_ids(void *h, uint32_t *ids, int n) {
    if (!h || !ids || n < 0) return -1;
    return guarded("wavec_gpu_get_ids", [&] {
        auto *ex = exec_or_throw(h);
        if ((uint32_t)n > ex->id_tokens) throw std::runtime_error("more ids than plan tokens");
        K44_HIP(hipMemcpyAsync(ids, ex->ids.p, (size_t)n * 4u, hipMemcpyDeviceToHost, ex->stream));
        K44_HIP(hipStreamSynchronize(ex->stream));
        return 0;
    });
}

int wavec_gpu_set_history(void *h, int steps) {
    if (!h || steps <= 0) return -1;
    return guarded("wavec_gpu_set_history", [&] {
        exec_or_throw(h)->set_history((uint32_t)steps);
        return 0;
    });
}

int wavec_gpu_get_history(void *h, uint32_t *out, int n) {
    if (!h || !out || n < 0) return -1;
    return guarded("wavec_gpu_get_history", [&] {
        auto *ex = exec_or_throw(h);
        if (!ex->hist_steps) throw std::runtime_error("no history buffer (wavec_gpu_set_history)");
        uint32_t steps = 0;
        K44_HIP(hipMemcpyAsync(&steps, ex->step_ctr.p, 4u, hipMemcpyDeviceToHost, ex->stream));
        K44_HIP(hipStreamSynchronize(ex->stream));
        const size_t avail = (size_t)std::min(steps, ex->hist_steps) * ex->id_tokens;
        const size_t cnt = std::min(avail, (size_t)n);
        if (cnt)
            K44_HIP(hipMemcpyAsync(out, ex->history.p, cnt * 4u, hipMemcpyDeviceToHost, ex->stream));
        K44_HIP(hipStreamSynchronize(ex->stream));
        return (int)std::min(steps, ex->hist_steps);
    });
}

int wavec_gpu_use_graph(void *h, int enable) {
    if (!h) return -1;
    return guarded("wavec_gpu_use_graph", [&] {
        auto *ex = exec_or_throw(h);
        K44_HIP(hipStreamSynchronize(ex->stream));
        ex->use_graph = enable != 0;
        if (!ex->use_graph) ex->drop_graph();
        return 0;
    });
}

int wavec_gpu_copy_canvas(void *dst_h, unsigned long long dst_off, void *src_h,
                          unsigned long long src_off, unsigned long long n) {
    if (!dst_h || !src_h) return -1;
    return guarded("wavec_gpu_copy_canvas", [&] {
        auto *d = exec_or_throw(dst_h);
        auto *s = exec_or_throw(src_h);
        if (dst_off > d->plan_meta.canvas_elems || n > d->plan_meta.canvas_elems - dst_off ||
            src_off > s->plan_meta.canvas_elems || n > s->plan_meta.canvas_elems - src_off)
            throw std::runtime_error("range outside a canvas");
        K44_HIP(hipStreamSynchronize(s->stream));
        K44_HIP(hipMemcpyAsync(d->canvas.p + dst_off, s->canvas.p + src_off, n * 2u,
                               hipMemcpyDeviceToDevice, d->stream));
        K44_HIP(hipStreamSynchronize(d->stream));
        return 0;
    });
}

int wavec_gpu_copy_ids(void *dst_h, int dst_first, void *src_h, int src_first, int src_step,
                       int n) {
    if (!dst_h || !src_h || dst_first < 0 || src_first < 0 || src_step <= 0 || n < 0) return -1;
    return guarded("wavec_gpu_copy_ids", [&] {
        auto *d = exec_or_throw(dst_h);
        auto *s = exec_or_throw(src_h);
        if ((uint64_t)dst_first + n > d->id_tokens ||
            (n && (uint64_t)src_first + (uint64_t)(n - 1) * src_step >= s->id_tokens))
            throw std::runtime_error("id range outside a plan's token-id buffer");
        K44_HIP(hipStreamSynchronize(s->stream));
        K44_HIP(hipMemcpy2DAsync(d->ids.p + dst_first, 4u, s->ids.p + src_first,
                                 (size_t)src_step * 4u, 4u, (size_t)n, hipMemcpyDeviceToDevice,
                                 d->stream));
        K44_HIP(hipStreamSynchronize(d->stream));
        return 0;
    });
}

const char *wavec_gpu_exec_report_json(void *h) {
    k44_host::K44GpuExecutorState *ex = h ? k44_host::find_exec(h) : nullptr;
    return ex ? ex->report_json.c_str() : "{}";
}

int wavec_gpu_execute_runs(void *h, int first_run, int n_runs) {
    if (!h || first_run < 0 || n_runs < 0) return -1;
    return guarded("wavec_gpu_execute_runs", [&] {
        auto *ex = exec_or_throw(h);
        if ((size_t)first_run + (size_t)n_runs > ex->runs.size())
            throw std::runtime_error("run range past the end of the plan's schedule");
        ex->launch_ops((size_t)first_run, (size_t)n_runs);
        K44_HIP(hipStreamSynchronize(ex->stream));
        return 0;
    });
}

int wavec_gpu_read_canvas_2d(void *h, unsigned long long off, unsigned long long rows,
                             unsigned long long row_stride, unsigned long long cols,
                             uint16_t *dst) {
    if (!h || (!dst && rows && cols)) return -1;
    return guarded("wavec_gpu_read_canvas_2d", [&] {
        auto *ex = exec_or_throw(h);
        if (!rows || !cols) return 0;
        // Anything inside the allocation may be read (relocated multiply operands live past
        // the plan's canvas).
        const uint64_t n = ex->canvas.n;
        if (cols > row_stride || off > n || rows - 1u > (n - off) / row_stride ||
            off + (rows - 1u) * row_stride + cols > n)
            throw std::runtime_error("2-D range outside the canvas allocation");
        // Packed on the device first (a staging buffer kept by the executor), then one copy.
        if (ex->stage.n < rows * cols) ex->stage.alloc(rows * cols);
        K44_HIP(k44dev::launch_gather_cols(ex->stage.p,
                                           reinterpret_cast<const uint16_t *>(ex->canvas.p + off),
                                           rows, row_stride, cols, ex->stream));
        K44_HIP(hipMemcpyAsync(dst, ex->stage.p, rows * cols * 2u, hipMemcpyDeviceToHost,
                               ex->stream));
        K44_HIP(hipStreamSynchronize(ex->stream));
        return 0;
    });
}

int wavec_set_tuning(const char *key, int value) {
    if (!key) return -1;
    return guarded("wavec_set_tuning", [&] {
        for (int i = 0; i < (int)k44_host::Tune::Count; ++i) {
            if (std::string(key) != k44_host::kTuneKeys[i]) continue;
            const k44_host::TuneValues &tv = k44_host::kTuneValues[i];
            const bool ok = value == -1 || (tv.set ? (value >= 0 && value < 32 &&
                                                      ((tv.set >> value) & 1u))
                                                   : value >= tv.min);
            if (!ok) {
                std::string allowed;
                if (tv.set) {
                    for (int v = 0; v < 32; ++v)
                        if ((tv.set >> v) & 1u) allowed += (allowed.empty() ? "" : " | ") + std::to_string(v);
                } else {
                    allowed = ">= " + std::to_string(tv.min);
                }
                throw std::runtime_error(std::string("value ") + std::to_string(value) +
                                         " is not honoured by '" + key + "' (-1 or " + allowed + ")");
            }
            k44_host::g_tune[i].store(value);
            return 0;
        }
        throw std::runtime_error(std::string("unknown tuning key '") + key + "'");
    });
}

int wavec_get_tuning(const char *key) {
    if (!key) return -2;
    for (int i = 0; i < (int)k44_host::Tune::Count; ++i)
        if (std::string(key) == k44_host::kTuneKeys[i]) return k44_host::g_tune[i].load();
    set_error(std::string("wavec_get_tuning: unknown tuning key '") + key + "'");
    return -2;
}

void wavec_reset_tuning(void) {
    for (auto &v : k44_host::g_tune) v.store(-1);
}

}  // extern "C"
