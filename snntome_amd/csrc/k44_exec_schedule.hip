// Executor: fusion of token ops into waves, whole-plan scheduling, the persistent decode
// program and the execution report (see k44_executor.hpp).
#include "k44_executor.hpp"

namespace k44_host {

void K44GpuExecutorState::drop_program(const std::string &why) {
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
void K44GpuExecutorState::build_program() {
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
void K44GpuExecutorState::check_program() {
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

// Canvas ranges an aux command reads and writes (the 2-D commands: everything).
void K44GpuExecutorState::aux_ranges(const AuxExec &a, Ranges &rd, Ranges &wr) const {
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
void K44GpuExecutorState::fuse_products() {
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
void K44GpuExecutorState::fuse_mul_chains() {
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
void K44GpuExecutorState::fuse_norm_shifts() {
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

// A decode RMSNorm that runs its token shift (fuse_norm_shifts) and whose producers store the
// sums of squares is not launched either when every reader of the shift's output is a narrow
// 64/128-neuron wave gathering it plainly: those waves gather the norm's input and apply the
// norm and the shift in their gather (gather form 5, the norm and shift kernel's expressions).
// The state update cannot happen there in place (other workgroups of the same launch read the
// old state): for every channel one reading workgroup stores the shifted state in a private
// buffer (shift_next), and the workgroups of the next narrow launch after the last reader (the
// carrier) copy it back.  Conditions: a decode shift with 2 <= rf <= 4 and a state; the norm's
// output read by nothing else and the shift's output only by such waves (segments inside it, at
// the canvas step of its rows) until overwritten, neither the plan output; the norm's input
// intact until the last reader; nothing from the norm to the carrier touching the state; every
// channel gathered by some reader; contraction chunks of at most 4 sub-chunks (64 k-steps).
// Returns the readers, the carrier (index into ops) and per reader the ownership bits of its
// work items (MfmaTileArgs::own).
bool K44GpuExecutorState::fold_shift(size_t i, const std::pair<uint64_t, uint64_t> &X,
                                     const std::pair<uint64_t, uint64_t> &Y,
                                     const std::vector<Ranges> &rd, const std::vector<Ranges> &wr,
                                     const Ranges &out_rng, std::vector<size_t> &cons,
                                     size_t &refresher, size_t &carrier,
                                     std::vector<std::vector<uint64_t>> &owns,
                                     size_t embed_aux) {
    typedef std::pair<uint64_t, uint64_t> Rng;
    const AuxExec &N = *aux[ops[i].second];
    const AuxExec &T = *aux[N.shift_with];
    if (!T.decode || T.rf < 2u || T.rf > 4u || !T.has_state || T.tokens != N.tokens ||
        T.stride != N.stride || T.D != N.D || T.tokens > 16u)
        return false;
    const uint64_t D = N.D, stride = N.stride;
    const Rng Sg(T.y_off, T.y_off + D * stride);
    const Rng St(T.state_off, T.state_off + D * (T.rf - 1u) * 64u);
    auto narrow_long = [&](const WaveExec &w) {
        return w.mfma && w.narrow && (w.cluster == 64u || w.cluster == 128u) && !w.tile2d;
    };
    const size_t n = ops.size();
    cons.clear();
    size_t last = i;
    bool ow_y = false, ow_s = false;
    for (size_t j = i + 1; j < n && !(ow_y && ow_s); ++j) {
        if (!ow_y && ranges_overlap(rd[j], Ranges{Y})) return false;
        if (!ow_s && ranges_overlap(rd[j], Ranges{Sg})) {
            if (!ops[j].first) return false;
            const WaveExec &w = *waves[ops[j].second];
            bool ok = narrow_long(w) && w.xprod == 0u && w.step == stride && w.S % 32u == 0u &&
                      !ranges_overlap(w.resrd, Ranges{Sg}) &&
                      (w.kgroups > 1u ? w.stage_chunk : w.ksteps) <= 64u &&
                      w.seg_h.size() == (size_t)w.rows * w.K;
            for (const auto &x : w.xrd) ok = ok && Sg.first <= x.first && x.second <= Sg.second;
            if (!ok) return false;
            cons.push_back(ops[j].second);
            last = j;
        }
        ow_y = ow_y || ranges_overlap(wr[j], Ranges{Y});
        ow_s = ow_s || ranges_overlap(wr[j], Ranges{Sg});
    }
    if (cons.empty() || (!ow_y && ranges_overlap(Ranges{Y}, out_rng)) ||
        (!ow_s && ranges_overlap(Ranges{Sg}, out_rng)))
        return false;
    for (size_t j = i + 1; j <= last; ++j)
        if (ranges_overlap(wr[j], Ranges{X})) return false;
    carrier = SIZE_MAX;
    for (size_t j = last + 1; j < n && carrier == SIZE_MAX; ++j)
        if (ops[j].first && narrow_long(*waves[ops[j].second]) &&
            waves[ops[j].second]->cp_fold == SIZE_MAX)
            carrier = j;
    if (carrier == SIZE_MAX) return false;
    for (size_t j = i + 1; j <= carrier; ++j)
        if (ranges_overlap(rd[j], Ranges{St}) || ranges_overlap(wr[j], Ranges{St})) return false;
    // the refresher: the last narrow launch before the norm, or else the decode embedding that
    // produces the norm's input (embed_aux), with nothing after it writing the state before the
    // readers
    refresher = SIZE_MAX;
    for (size_t j = i; j-- > 0 && refresher == SIZE_MAX;)
        if (ops[j].first && narrow_long(*waves[ops[j].second]) &&
            waves[ops[j].second]->cp_fold == SIZE_MAX)
            refresher = j;
    if (refresher == SIZE_MAX && embed_aux != SIZE_MAX && aux[embed_aux]->cp_fold == SIZE_MAX)
        for (size_t j = i; j-- > 0 && refresher == SIZE_MAX;)
            if (!ops[j].first && ops[j].second == embed_aux) refresher = j;
    if (refresher == SIZE_MAX) return false;
    for (size_t j = refresher; j < i; ++j)
        if (ranges_overlap(wr[j], Ranges{St})) return false;
    // ownership: the first work item (readers in plan order, items in launch order) gathering a
    // channel not yet covered stores the shifted state of its pass (a channel stored twice gets
    // the same bits twice)
    std::vector<uint8_t> cov(D, 0u);
    uint64_t ncov = 0;
    owns.assign(cons.size(), {});
    for (size_t k = 0; k < cons.size(); ++k) {
        const WaveExec &w = *waves[cons[k]];
        std::vector<uint64_t> &own = owns[k];
        own.assign((size_t)w.rows * w.kgroups, 0u);
        const uint32_t chunk = w.kgroups > 1u ? w.stage_chunk : w.ksteps;
        for (uint32_t z = 0; z < w.kgroups; ++z)
            for (uint32_t tl = 0; tl < w.rows; ++tl) {
                const uint32_t kb0 = z * chunk, ke = std::min(w.ksteps, kb0 + chunk);
                for (uint32_t s = 0; kb0 + 16u * s < ke; ++s) {
                    const uint32_t kb = kb0 + 16u * s, nr = (std::min(ke, kb + 16u) - kb) * 32u;
                    for (uint32_t p = 0; p < 16u && 32u * p < nr; ++p) {
                        const uint32_t r = kb * 32u + 32u * p, kk = r / w.S;
                        const uint64_t off = w.seg_h[(size_t)tl * w.K + kk] +
                                             (uint64_t)(r - kk * w.S) * w.step;
                        if (off < Sg.first || (off - Sg.first) % stride != 0u) return false;
                        const uint64_t c0 = (off - Sg.first) / stride;
                        bool fresh = false;
                        for (uint64_t c = c0; c < c0 + 32u && c < D; ++c)
                            if (!cov[c]) {
                                cov[c] = 1u;
                                ++ncov;
                                fresh = true;
                            }
                        if (fresh) own[(size_t)z * w.rows + tl] |= 1ull << (s * 16u + p);
                    }
                }
            }
    }
    return ncov == D;
}

// RMSNorms of decode-sized plans whose input is written by narrow 64/128-neuron MFMA waves
// (the sub-waves of the projections before them, each tile's outputs stored by one
// workgroup) take their per-token scales from those waves: every producer tile stores the
// exact sums of squares of the values it stored in a slot of its own (k44_mfma_narrow.hip,
// narrow_norm_publish), and each reader of the norm, in a later launch, adds all slots at its
// start, while its weight stream is in flight (rms_inv_from_slots).  The sums are exact, so
// the scales equal the norm kernel's own bit for bit.  A norm read only by narrow 64/128-neuron waves gathering
// it plainly is then not launched: those waves gather its input and normalise it in the
// gather with the kernel's expression (xprod 4).  Otherwise (a norm that runs the decode
// token shift) the norm kernel runs with the scales and skips its sum pass.  Conditions, from
// the canvas ranges of the commands in plan order: the producers are the last writers of
// the input, together write each of its D rows exactly once, and run their whole epilogue
// in one workgroup per tile (unsplit, or split-K reduced in the launch); for the consumers,
// the input stays intact until the last of them, and the norm's output is not the plan
// output.  Whole-plan execution only; tuning switch fuse=0 disables it.
void K44GpuExecutorState::fuse_norms() {
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
        size_t prod_embed = SIZE_MAX;  // or the decode embedding that writes all of X
        std::vector<uint8_t> row_seen(N.D, 0u);
        uint32_t covered = 0;
        bool ok = true;
        for (size_t p = i; p-- > 0 && ok && covered < N.D;) {
            if (!ranges_overlap(wr[p], Ranges{X})) continue;
            if (!ops[p].first) {
                const AuxExec &E = *aux[ops[p].second];
                // (k44_embed_vec_kernel's slot form: one 64-token block of <= 16 tokens, 64-
                // channel blocks, 16-byte rows; not with the persistent launch)
                ok = covered == 0u && E.type == K44CmdType::EMBED_1D && !E.fused &&
                     E.y_off == X.first && E.D == N.D && E.stride == 64u && N.stride == 64u &&
                     E.tokens <= 16u && E.tokens > 0u && E.D % 64u == 0u && E.y_off % 8u == 0u &&
                     E.slot_fold == SIZE_MAX && tune(Tune::Program) != 1;
                if (ok) {
                    prod_embed = ops[p].second;
                    covered = N.D;
                }
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
        if (!ok || covered != N.D || (prods.empty() && prod_embed == SIZE_MAX)) continue;
        // consumers (a norm without a fused shift): readers of Y until overwritten
        std::vector<size_t> cons;
        bool consume = N.shift_with == SIZE_MAX;
        // a norm with its decode token shift: the shift's readers (fold_shift below)
        size_t refresher = SIZE_MAX, carrier = SIZE_MAX;
        std::vector<std::vector<uint64_t>> owns;
        const bool shifted =
            !consume && tune(Tune::Program) != 1 &&
            fold_shift(i, X, Y, rd, wr, out_rng, cons, refresher, carrier, owns,
                       tune(Tune::EmbedRefresh) != 0 ? prod_embed : SIZE_MAX);
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
        if (prod_embed != SIZE_MAX) {
            AuxExec &E = *aux[prod_embed];
            E.slot_fold = norm_folds.size();
            E.slot_tile0 = f.tiles;
            f.tiles += E.D / 64u;
        }
        f.consumers = consume || shifted;
        N.norm_fold = norm_folds.size();
        if (shifted) {
            const AuxExec &T = *aux[N.shift_with];
            const Rng Sg(T.y_off, T.y_off + (uint64_t)T.D * T.stride);
            const Rng St(T.state_off, T.state_off + (uint64_t)T.D * (T.rf - 1u) * 64u);
            f.shift = N.shift_with;
            f.next0 = shift_next_elems;
            f.cur0 = f.next0 + (size_t)T.D * (T.rf - 1u) * 16u;
            shift_next_elems += 2u * (size_t)T.D * (T.rf - 1u) * 16u;
            N.fused = true;
            N.fuse_note = "folded with its token shift: sums of squares stored by its producers, "
                          "rows normalised and shifted in its readers' gathers";
            for (size_t k = 0; k < cons.size(); ++k) {
                WaveExec &w = *waves[cons[k]];
                w.xprod = 5u;
                w.xnorm = norm_folds.size();
                w.xd[0] = (int64_t)X.first - (int64_t)Sg.first;
                w.own.upload(owns[k]);
                Ranges fr = w.resrd;
                for (const auto &x : w.xrd)
                    fr.push_back({(uint64_t)((int64_t)x.first + w.xd[0]),
                                  (uint64_t)((int64_t)x.second + w.xd[0])});
                fr.push_back(St);
                w.rd_run = merge_ranges(std::move(fr));
                w.why += "; gathers its input through a folded RMSNorm and decode token shift";
            }
            // the compact copy is refreshed by the refresher's launch and the state written back
            // by the carrier's (neither grouped with a reader)
            if (ops[refresher].first) {
                WaveExec &rw = *waves[ops[refresher].second];
                rw.cp_fold = norm_folds.size();
                rw.cp_refresh = true;
                rw.carry_rng = {St};
                rw.why += "; its workgroups refresh the compact state copy of a later token shift";
            } else {
                aux[ops[refresher].second]->cp_fold = norm_folds.size();
            }
            WaveExec &cw = *waves[ops[carrier].second];
            cw.cp_fold = norm_folds.size();
            cw.carry_rng = {St};
            cw.why += "; its workgroups copy back the shifted state of an earlier token shift";
        } else if (consume) {
            N.fused = true;
            N.fuse_note = "folded: sums of squares stored by its producers, rows normalised "
                          "in its readers' gathers";
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
            N.fuse_note = "sums of squares stored by its producers (no sum pass)";
        }
        norm_folds.push_back(f);
    }
}

// Plan order -> runs: consecutive MFMA waves of one kernel configuration join a group while
// no member writes what another reads or writes (checked on canvas element ranges).
void K44GpuExecutorState::form_runs() {
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
                // (a carried state copy writes carry_rng)
                indep = !ranges_overlap(w.wr_run, o.rd_run) &&
                        !ranges_overlap(w.rd_run, o.wr_run) &&
                        !ranges_overlap(w.wr_run, o.wr_run) &&
                        !ranges_overlap(w.carry_rng, o.rd_run) &&
                        !ranges_overlap(w.carry_rng, o.wr_run) &&
                        !ranges_overlap(w.rd_run, o.carry_rng) &&
                        !ranges_overlap(w.wr_run, o.carry_rng);
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

size_t K44GpuExecutorState::launches_per_run() const {
    size_t n = 0;
    for (const auto &r : runs) {
        if (r.first == 2) n += groups[r.second]->epi_items ? 2u : 1u;
        else if (r.first == 0 && aux[r.second]->type == K44CmdType::ARGMAX_1D)
            n += hist_steps ? 3u : 2u;
        else n += 1u;
    }
    return n;
}

void K44GpuExecutorState::build_report() {
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
          << ", \"reduce_xcd_local\": " << (w.red_local ? "true" : "false")
          << ", \"flops\": " << (long long)w.flops
          << ", \"effective_flops\": " << (long long)w.eff_flops
          << ", \"mapped\": " << (w.cmap.p ? "true" : "false")
          << ", \"unique_rows\": " << w.unique_rows
          << ", \"y_off\": " << w.y_off << ", \"y_off_run\": " << w.y_off_run
          << ", \"xd\": [" << w.xd[0] << ", " << w.xd[1] << ", " << w.xd[2] << "]"
          // gather form 5: the token-shift command it applies; a carrier: the token-shift
          // command whose shifted state its launch copies back (-1: none)
          << ", \"shift_cmd\": "
          << (w.xprod == 5u ? (long long)aux_cmd[norm_folds[w.xnorm].shift] : -1LL)
          << ", \"copies_state_of\": "
          << (w.cp_fold != SIZE_MAX && !w.cp_refresh
                  ? (long long)aux_cmd[norm_folds[w.cp_fold].shift] : -1LL)
          << ", \"refreshes_state_of\": "
          << (w.cp_fold != SIZE_MAX && w.cp_refresh
                  ? (long long)aux_cmd[norm_folds[w.cp_fold].shift] : -1LL)
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
          << ", \"refreshes_state_of\": "
          << (aux[i]->cp_fold != SIZE_MAX ? (long long)aux_cmd[norm_folds[aux[i]->cp_fold].shift]
                                          : -1LL)
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
    o << "], \"launches_per_run\": " << (prog_active ? (size_t)1u : launches_per_run())
      << ", \"xcd_local_ok\": " << (xcd_local_ok ? "true" : "false");
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

}  // namespace k44_host
