// Executor: kernel launches, whole-plan execution and host I/O (see k44_executor.hpp).
#include "k44_executor.hpp"

namespace k44_host {

// whole: whole-plan execution (folded / fused commands apply).
void K44GpuExecutorState::launch_aux(const AuxExec &a, bool whole) {
    __half *cv = canvas.p;
    switch (a.type) {
    case K44CmdType::RMSNORM_1D:
        if (whole && a.shift_with != SIZE_MAX) {
            const AuxExec &t = *aux[a.shift_with];
            const k44dev::RmsShift sh{cv + t.y_off, t.table.p,
                                      t.has_state ? cv + t.state_off : nullptr, t.rf, 0u,
                                      t.decode ? 0u : t.seq_len};
            const uint64_t *sl = a.norm_fold != SIZE_MAX ? fold_slots(a.norm_fold) : nullptr;
            const uint32_t n = a.norm_fold != SIZE_MAX ? norm_folds[a.norm_fold].tiles : 0u;
            K44_HIP(k44dev::launch_rmsnorm(cv + a.y_off, cv + a.src_off, a.table.p, a.D,
                                           a.stride, a.tokens, a.eps, stream, &sh, sl, n));
        } else if (whole && a.norm_fold != SIZE_MAX) {
            K44_HIP(k44dev::launch_rmsnorm(cv + a.y_off, cv + a.src_off, a.table.p, a.D,
                                           a.stride, a.tokens, a.eps, stream, nullptr,
                                           fold_slots(a.norm_fold), norm_folds[a.norm_fold].tiles));
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
    case K44CmdType::EMBED_1D: {
        k44dev::EmbedCopy cp;
        if (whole && a.cp_fold != SIZE_MAX) {  // the first layer's compact token-shift state
            const NormFold &f = norm_folds[a.cp_fold];
            const AuxExec &T = *aux[f.shift];
            cp.src = cv + T.state_off;
            cp.sstride = 64u;
            cp.dst = shift_next.p + f.cur0;
            cp.dstride = 16u;
            cp.rows = T.D * (T.rf - 1u);
        }
        K44_HIP(k44dev::launch_embed(
            cv + a.y_off, a.table.p, ids.p, a.D, a.vocab, a.stride, a.tokens, stream,
            whole && a.slot_fold != SIZE_MAX
                ? reinterpret_cast<uint64_t *>(norm_slots.p) +
                      (norm_folds[a.slot_fold].slot0 + a.slot_tile0) * 32u
                : nullptr,
            cp));
        break;
    }
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

void K44GpuExecutorState::launch_mfma_group(const k44dev::MfmaGroup &d, uint32_t nt, uint32_t mt, uint32_t rows,
                       uint32_t items, uint32_t epi_items, bool dma, const k44dev::DmaShape &ds,
                       uint32_t prod, uint32_t max_items, bool mis,
                       const k44dev::NarrowPre &pre) {
    if (mt == 16u)  // narrow (<= 16 tokens)
        K44_HIP(k44dev::launch_mfma_narrow(d, nt, items, stream, prod, max_items, pre));
    else if (dma)
        K44_HIP(k44dev::launch_mfma_dma(d, nt, items, stream, ds));
    else
        K44_HIP(k44dev::launch_mfma_tile(d, nt, mt, rows, items, stream, mis));
    if (epi_items) K44_HIP(k44dev::launch_splitk_epilogue(d, epi_items, stream));
}

void K44GpuExecutorState::launch_mfma(const WaveExec &w) {
    const k44dev::MfmaGroup d{w.one_args.p, w.one_start.p, 1u, xcd_order};
    launch_mfma_group(d, w.cluster, w.mt, w.rows_per_stage, w.items, w.epi_items, w.dma,
                      w.dshape, 0u, w.items, w.mis, w.one_pre);
}

void K44GpuExecutorState::launch_group(const MfmaGroupExec &g) {
    const k44dev::MfmaGroup d{g.args.p, g.start.p, (uint32_t)g.members.size(), xcd_order};
    launch_mfma_group(d, g.nt, g.mt, g.rows, g.items, g.epi_items, g.dma, g.dshape,
                      g.prod, g.max_items, g.mis, g.pre);
}

void K44GpuExecutorState::launch_wave(const WaveExec &w) {
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

void K44GpuExecutorState::launch_op(size_t i) {
    const auto &op = ops.at(i);
    if (op.first)
        launch_wave(*waves[op.second]);
    else
        launch_aux(*aux[op.second]);
}

void K44GpuExecutorState::launch_ops(size_t first, size_t n) {
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
void K44GpuExecutorState::execute_plan() {
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

void K44GpuExecutorState::set_history(uint32_t steps) {
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

void K44GpuExecutorState::upload_input_f32(const float *in, size_t n) {
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

std::vector<float> K44GpuExecutorState::download_output_f32() {
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

int K44GpuExecutorState::infer_f32(const float *in, int in_elems, float *out, int out_elems, float *ms_out) {
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

}  // namespace k44_host
