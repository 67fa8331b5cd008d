// Executor: plan validation and device upload (see k44_executor.hpp).
#include "k44_executor.hpp"

namespace k44_host {

void K44GpuExecutorState::drop_graph() {
    if (graph_exec) (void)hipGraphExecDestroy(graph_exec);
    if (graph) (void)hipGraphDestroy(graph);
    graph_exec = nullptr;
    graph = nullptr;
}

void K44GpuExecutorState::free_all() {
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
    shift_next.reset();
    shift_mix.reset();
    shift_next_elems = 0;
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
void K44GpuExecutorState::segment_rows(const K44ExecCmd &c, uint64_t step, uint32_t &S_out,
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
bool K44GpuExecutorState::streaming_gather(const WaveExec &wx) {
    if (tune(Tune::NonTemporal) >= 0) return tune(Tune::NonTemporal) == 1;
    return wx.unique_rows * (uint64_t)wx.tokens * 2u >= (512ull << 20);
}

// MFMA configuration of a wave with a dense tiling (tiles of cl = cluster_size neurons
// sharing every index row): kernel (narrow <= 16 tokens, LDS ring for 512-token
// workgroups, register-staged tile otherwise), ring depth, split-K, and the weights in
// A-fragment order.  width: the output's token count per row (1-D waves; 2-D waves pass
// UINT32_MAX: they never take the narrow kernel).
void K44GpuExecutorState::configure_mfma(const K44ExecCmd &c, WaveExec &wx, const std::vector<uint16_t> &wraw,
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
            // in 16-k-step sub-chunks.  Chunks of at most 32 k-steps; split further, down
            // to 16 k-steps, until the wave has ~64 workgroups (~128 when a second kernel
            // reduces the partials).  Measured on config-5 decode (ms per step, graph
            // replays, alternated in one process): partials reduced by the tile's last
            // workgroup 0.869 at 64 workgroups, 0.889 at 32, 0.941 at 128, 0.968 unsplit
            // beyond 48 k-steps; reduced by the epilogue kernel 0.928 at 128 or 64.  With
            // the folded norms and token shifts, at most 32 k-steps per chunk: 0.7685 against
            // 0.7896 at 48, 0.787 at 40, 0.829 at 24, 0.841 at 16 (the down projections'
            // 96-k-step contractions in 3 chunks instead of 2: each workgroup's weights two
            // 16-k-step round trips instead of three).
            const int ce = tune(Tune::NarrowChunk), cw = tune(Tune::NarrowWgs);
            const uint32_t cmax = ce > 0 ? (uint32_t)std::max(16, ce) : 32u;
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

void K44GpuExecutorState::build_wave(const K44ExecCmd &c, WaveExec &wx) {
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
    if (wx.narrow) wx.seg_h = starts;
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
void K44GpuExecutorState::build_wave2d(const K44ExecCmd &c, WaveExec &wx, const K44ResDesc &Lo,
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
void K44GpuExecutorState::build_spatial(const K44ExecCmd &c, AuxExec &ax) {
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

void K44GpuExecutorState::build_aux(const K44ExecCmd &c, AuxExec &ax) {
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

void K44GpuExecutorState::init(const K44WavePlan &plan) {
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
        // Meetings through one XCD's L2 (the chunks of a tile 8 workgroups apart in launch
        // order; partial offsets below 2 GiB), their counters one 128-byte line per tile.
        bool need = false;
        for (auto &wp : waves) need = need || wp->reduce_in_kernel;
        if (need && tune(Tune::NarrowLocal) != 0) probe_xcd_placement();
        n_arrive = 0;
        for (auto &wp : waves)
            if (wp->reduce_in_kernel) {
                wp->red_local = xcd_local_ok &&
                                (uint64_t)wp->kgroups * wp->cout * 64u < (1ull << 31);
                any_local = any_local || wp->red_local;
                wp->arrive_off = n_arrive;
                n_arrive += (size_t)wp->rows * (wp->red_local ? 32u : 1u);
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
        K44_HIP(hipMemsetAsync(norm_slots.p, 0, slots * 64u * sizeof(uint32_t), stream));
        if (shift_next_elems) {
            shift_next.alloc(shift_next_elems);
            K44_HIP(hipMemsetAsync(shift_next.p, 0, shift_next_elems * sizeof(__half), stream));
            // per folded token shift: [D][8] = mu[c][0..rf-1], 0 .., the norm's gamma at 4
            std::vector<__half> mix;
            for (NormFold &f : norm_folds) {
                if (f.shift == SIZE_MAX) continue;
                const AuxExec &T = *aux[f.shift], &N = *aux[f.norm];
                std::vector<uint16_t> mu((size_t)T.D * T.rf), gm(N.D, 0x3c00u);
                K44_HIP(hipMemcpy(mu.data(), T.table.p, mu.size() * 2u, hipMemcpyDeviceToHost));
                if (N.table.p)
                    K44_HIP(hipMemcpy(gm.data(), N.table.p, gm.size() * 2u, hipMemcpyDeviceToHost));
                f.mix0 = mix.size();
                std::vector<uint16_t> rows((size_t)T.D * 8u, 0u);
                for (size_t c = 0; c < T.D; ++c) {
                    for (uint32_t i = 0; i < T.rf; ++i) rows[c * 8u + i] = mu[c * T.rf + i];
                    rows[c * 8u + 4u] = gm[c];
                }
                mix.resize(mix.size() + rows.size());
                std::memcpy(mix.data() + f.mix0, rows.data(), rows.size() * 2u);
            }
            shift_mix.upload(mix);
        }
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

// Contraction split of an MFMA wave into `want` chunks (k-steps for the narrow kernels,
// stages of rows_per_stage positions otherwise).
void K44GpuExecutorState::set_split(WaveExec &w, uint32_t want) {
    const uint32_t units = w.narrow ? w.ksteps : w.K * w.S / w.rows_per_stage;
    want = std::max(1u, std::min(want, units));
    w.stage_chunk = (units + want - 1u) / want;
    w.kgroups = (units + w.stage_chunk - 1u) / w.stage_chunk;
    w.part_floats = w.kgroups > 1u ? (size_t)w.kgroups * w.cout * w.part_tokens : 0u;
}

k44dev::MfmaTileArgs K44GpuExecutorState::mfma_args(const WaveExec &w, float *part, bool fused) const {
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
    if (fused && w.reduce_in_kernel) {
        a.arrive = arrive.p + w.arrive_off;
        a.red_local = w.red_local ? 1u : 0u;
    }
    if (fused && w.norm_fold != SIZE_MAX) {
        const NormFold &f = norm_folds[w.norm_fold];
        a.norm_part = norm_slots.p + (f.slot0 + w.norm_tile0) * 64u;
    }
    if (fused && w.xnorm != SIZE_MAX) {
        const NormFold &f = norm_folds[w.xnorm];
        const AuxExec &N = *aux[f.norm];
        a.xslots = norm_slots.p + f.slot0 * 64u;
        a.xslots_n = f.tiles;
        a.norm_D = N.D;
        a.norm_eps = N.eps;
        a.xgamma = N.table.p;
        a.xg_base = N.y_off;
        uint32_t sh = 0;
        while ((1u << sh) < N.stride) ++sh;
        a.xg_shift = sh;
        if (w.xprod == 5u) {  // rows of the shift's output; its mixing weights and state
            const AuxExec &T = *aux[f.shift];
            a.xg_base = T.y_off;
            a.mixg = shift_mix.p + f.mix0;
            a.state = shift_next.p + f.cur0;
            a.state_next = shift_next.p + f.next0;
            a.own = w.own.p;
            a.rf = T.rf;
            a.sh_tokens = T.tokens;
        }
    }
    if (fused && w.cp_fold != SIZE_MAX) {  // a folded token shift's state copy (16 tokens)
        const NormFold &f = norm_folds[w.cp_fold];
        const AuxExec &T = *aux[f.shift];
        a.cp_rows = T.D * (T.rf - 1u);
        if (w.cp_refresh) {  // the plan's state into the readers' compact copy
            a.cp_src = canvas.p + T.state_off;
            a.cp_sstride = 64u;
            a.cp_dst = shift_next.p + f.cur0;
            a.cp_dstride = 16u;
        } else {  // the shifted state back into the plan's
            a.cp_src = shift_next.p + f.next0;
            a.cp_sstride = 16u;
            a.cp_dst = canvas.p + T.state_off;
            a.cp_dstride = 64u;
        }
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

uint32_t K44GpuExecutorState::epi_workgroups(const WaveExec &w) {
    if (w.kgroups <= 1u) return 0u;
    return (uint32_t)(((uint64_t)w.cout * (w.part_tokens / 4u) + 255u) / 256u);
}

// Device descriptors: every MFMA wave alone (command-by-command runs) and every group.
void K44GpuExecutorState::upload_mfma_descriptors() {
    for (auto &wp : waves) {
        WaveExec &w = *wp;
        if (!w.mfma) continue;
        w.items = w.rows * (w.narrow ? 1u : w.tokens / w.mt) * w.kgroups;
        w.epi_items = epi_workgroups(w);
        const k44dev::MfmaTileArgs one = mfma_args(w, scratch.p, false);
        w.one_args.upload({one});
        w.one_start.upload({0u, w.items});
        w.one_pre = w.narrow ? narrow_pre({one}, {}, nullptr) : k44dev::NarrowPre{};
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
        // Narrow waves meeting XCD-locally number their items in groups of 8 tiles; with one in
        // the group, every wave's items start at a multiple of 8 (positions past a wave's own
        // items are idle).
        bool local = false;
        for (size_t m : order) local = local || waves[m]->red_local;
        for (size_t m : order) {
            const WaveExec &w = *waves[m];
            args.push_back(mfma_args(w, scratch.p ? scratch.p + off : nullptr, true));
            off += w.part_floats;
            uint32_t it = w.narrow ? k44dev::narrow_items(w.rows, w.kgroups, w.red_local) : w.items;
            if (local) it = (it + 7u) / 8u * 8u;
            start.push_back(start.back() + it);
            if (!w.reduce_in_kernel) epi_max = std::max(epi_max, w.epi_items);
            item_max = std::max(item_max, it);
        }
        g.items = start.back();
        g.epi_items = epi_max;  // epilogue grid: epi_max x members
        g.max_items = item_max;  // (0: narrow launches find each workgroup's wave by prefix sums)
        if (g.mt == 16u && tune(Tune::NarrowByy) == 0) g.max_items = 0u;
        if (xcd_order == 2u) check_balanced_order(start);
        g.args.upload(args);
        g.start.upload(start);
        if (g.mt == 16u) g.pre = narrow_pre(args, order, &g.pre_w);
    }
}

// Where workgroups run: probe launches of 4,096 and 1,001 workgroups record the XCD of each.
// The XCD-local split-K meeting needs workgroups a multiple of 8 apart in one launch to share an
// XCD (the round-robin dispatch over the 8 XCDs, or fewer in a partitioned mode).
void K44GpuExecutorState::probe_xcd_placement() {
    constexpr uint32_t n0 = 4096u, n1 = 1001u;
    DevBuf<uint32_t> out;
    out.alloc(n0 + n1);
    K44_HIP(k44dev::launch_xcd_probe(out.p, n0, stream));
    K44_HIP(k44dev::launch_xcd_probe(out.p + n0, n1, stream));
    std::vector<uint32_t> h(n0 + n1);
    K44_HIP(hipMemcpyAsync(h.data(), out.p, h.size() * 4u, hipMemcpyDeviceToHost, stream));
    K44_HIP(hipStreamSynchronize(stream));
    bool ok = true;
    for (uint32_t b = 8; b < n0 && ok; ++b) ok = h[b] == h[b % 8u];
    for (uint32_t b = 8; b < n1 && ok; ++b) ok = h[n0 + b] == h[n0 + b % 8u];
    xcd_local_ok = ok;
}

// Every XCD-local meeting leaves its tile's arrival counter at zero; a counter left nonzero
// means chunks of a tile ran on different XCDs and met no one.  Checked at each host
// synchronisation of a whole-plan run (the counters are then zeroed again).
void K44GpuExecutorState::check_placement() {
    if (!any_local || !n_arrive) return;
    std::vector<uint32_t> h(n_arrive);
    K44_HIP(hipMemcpyAsync(h.data(), arrive.p, n_arrive * 4u, hipMemcpyDeviceToHost, stream));
    K44_HIP(hipStreamSynchronize(stream));
    size_t bad = 0;
    for (uint32_t v : h) bad += v != 0u;
    if (!bad) return;
    K44_HIP(hipMemsetAsync(arrive.p, 0, n_arrive * 4u, stream));
    K44_HIP(hipStreamSynchronize(stream));
    throw std::runtime_error(std::to_string(bad) + " split-K arrival counters of XCD-local "
                             "reductions were left nonzero (chunks of a tile ran on different "
                             "XCDs); the outputs of that run are unreliable (tuning "
                             "narrow_local=0 avoids these reductions)");
}

// Weights and geometry of up to six descriptors for the narrow kernels' preloaded arguments
// (tuning key narrow_pre 0: none, every wave reads its descriptor).  One member: its own
// weights; several: copies of their A fragments in *arena, member m at m << shift bytes
// (shift: the largest member's bytes rounded up to a power of two).  members: the waves of
// args, in the same order.
k44dev::NarrowPre K44GpuExecutorState::narrow_pre(const std::vector<k44dev::MfmaTileArgs> &args,
                                                  const std::vector<size_t> &members,
                                                  DevBuf<__half> *arena) {
    k44dev::NarrowPre p;
    if (tune(Tune::NarrowPre) == 0 || args.empty()) return p;
    const size_t n = std::min(args.size(), (size_t)k44dev::NarrowPre::N);
    if (args.size() == 1u || !arena) {
        p.base = args[0].Wf;
        p.geo[0] = k44dev::narrow_geo(args[0]);
        return p;
    }
    size_t most = 256u;
    for (size_t i = 0; i < n; ++i) most = std::max(most, waves[members[i]]->w.n * sizeof(__half));
    uint32_t sh = 8u;
    while (((size_t)1 << sh) < most) ++sh;
    arena->alloc((n << sh) / sizeof(__half));
    for (size_t i = 0; i < n; ++i) {
        const WaveExec &w = *waves[members[i]];
        K44_HIP(hipMemcpyAsync(reinterpret_cast<char *>(arena->p) + (i << sh), w.w.p,
                               w.w.n * sizeof(__half), hipMemcpyDeviceToDevice, stream));
        p.geo[i] = k44dev::narrow_geo(args[i]);
    }
    K44_HIP(hipStreamSynchronize(stream));
    p.base = arena->p;
    p.shift = sh;
    return p;
}

// Stages (k-steps for the narrow kernels) one work item of an MFMA wave runs.
uint32_t K44GpuExecutorState::item_stages(const WaveExec &w) {
    const uint32_t units = w.narrow ? w.ksteps : w.K * w.S / w.rows_per_stage;
    return (units + w.kgroups - 1u) / w.kgroups;
}

// The per-wave XCD shares must be a bijection of the group's items (every item run by
// exactly one workgroup); checked on the host for every group before its first launch.
void K44GpuExecutorState::check_balanced_order(const std::vector<uint32_t> &start) {
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

}  // namespace k44_host
