// k44_wave_compiler.hpp — graph -> wave-plan compiler (namespace k44_host).
//
// Public API of the reference's K44WaveGraphCompiler (wavec/k44_wave_compiler.hpp): the add_*
// builders, compile() and the summary JSON.  The five passes are restated from the reference's
// documented behaviour so that the same graph yields the same plan (canvas offsets, index
// tables, weight blocks) and therefore the same .tcff bytes:
//   pass1_infer_shapes     shapes, auto-flatten of 2-D -> 1x1 linear           (ref :78-223)
//   pass2_fold_rmsnorm     RMSNorm gamma folded into 1x1 consumers            (ref :233-301)
//   pass3_build_layouts    resolution descriptors, wave configs               (ref :315-366)
//   pass4_allocate_canvas  liveness + best-fit interval allocator             (ref :388-593)
//   pass5_emit_commands    zero-copy views, K44_WAVE / aux command emission   (ref :824-988)
// Build extension: "SparseWave" nodes (add_sparse_wave / add_cluster_wave) — a wave whose
// neurons read explicit substrate positions (per-neuron or per-cluster index rows), which the
// reference's dense-only builders cannot express.  Canvas offsets are 64-bit; a sparse wave
// whose offsets do not fit the reference's u32 index words is emitted in row-index mode
// (K44ExecCmd::idx_mode = 1).
#pragma once
#include <algorithm>
#include <map>
#include <numeric>
#include <set>
#include <stdexcept>

#include "k44_plan_types.hpp"
#include "k44_tcff_io.hpp"

namespace k44_host {

// Distinct clusters up to which pruned projections take pack_union_tiles (2^12 masks).
constexpr uint32_t kMaxPackClusters = 12;

// Tiles of T neurons with small cluster unions for a pruned projection: pm[j] = neuron j's
// cluster set as a bit mask over nu <= kMaxPackClusters distinct clusters.  A tile's MFMA work
// (and, where all of a launch's work items run at once, the launch's time) grows with its
// union, so this bounds the largest union first.  Returns the tiles' neuron lists (each
// ascending), in creation order.
//  1. Greedy, one tile at a time: among the masks containing at least need = min(T, unassigned)
//     unassigned patterns (subset-sum transform of the pattern counts), the one with the fewest
//     clusters, then the most patterns, then the smallest mask value; of its unassigned neurons
//     the `need` that lie in the fewest other such masks (superset-sum transform), ties by index.
//  2. Swaps: while the first tile W with the largest union can drop one of its clusters c —
//     tried in order of (neurons of W using c, c) — by trading each of its neurons a that use c
//     (W's current list order) for the first neuron b (tiles in order, each tile's current list
//     in order) not yet traded, not using c, inside W's union, such that b's tile keeps a union
//     smaller than W's: trade them all (a to the end of b's tile, b to the end of W) and repeat,
//     at most max_iter times.
inline std::vector<std::vector<uint32_t>> pack_union_tiles(const std::vector<uint32_t> &pm,
                                                           uint32_t nu, uint32_t T,
                                                           uint32_t max_iter) {
    const uint32_t n = (uint32_t)pm.size(), NM = 1u << nu;
    std::vector<uint8_t> left(n, 1u);
    uint32_t n_left = n;
    std::vector<std::vector<uint32_t>> tiles;
    std::vector<int64_t> cnt(NM), v(NM);
    while (n_left) {
        const uint32_t need = std::min(T, n_left);
        std::fill(cnt.begin(), cnt.end(), 0);
        for (uint32_t j = 0; j < n; ++j)
            if (left[j]) ++cnt[pm[j]];
        for (uint32_t b = 0; b < nu; ++b)  // cnt[m] = unassigned patterns inside m
            for (uint32_t m = 0; m < NM; ++m)
                if (m >> b & 1u) cnt[m] += cnt[m ^ (1u << b)];
        uint32_t best = NM - 1u;  // the full mask holds every pattern
        for (uint32_t m = 0; m < NM; ++m) {
            if (cnt[m] < (int64_t)need) continue;
            const int pm_ = __builtin_popcount(m), pb = __builtin_popcount(best);
            if (pm_ < pb || (pm_ == pb && (cnt[m] > cnt[best] || (cnt[m] == cnt[best] && m < best))))
                best = m;
        }
        for (uint32_t m = 0; m < NM; ++m) v[m] = (cnt[m] >= (int64_t)need && m != best) ? 1 : 0;
        for (uint32_t b = 0; b < nu; ++b)  // v[m] = other such masks containing m
            for (uint32_t m = 0; m < NM; ++m)
                if (!(m >> b & 1u)) v[m] += v[m | (1u << b)];
        std::vector<uint32_t> mem;
        for (uint32_t j = 0; j < n; ++j)
            if (left[j] && (pm[j] & ~best) == 0u) mem.push_back(j);
        std::stable_sort(mem.begin(), mem.end(),
                         [&](uint32_t a, uint32_t b) { return v[pm[a]] < v[pm[b]]; });
        mem.resize(need);
        std::sort(mem.begin(), mem.end());
        for (uint32_t j : mem) left[j] = 0u;
        n_left -= need;
        tiles.push_back(std::move(mem));
    }
    const size_t nt = tiles.size();
    std::vector<std::vector<int64_t>> cc(nt, std::vector<int64_t>(nu, 0));  // neurons per cluster
    auto add = [&](size_t t, uint32_t mask, int64_t d) {
        for (uint32_t c = 0; c < nu; ++c)
            if (mask >> c & 1u) cc[t][c] += d;
    };
    auto usize = [&](const std::vector<int64_t> &x) {
        uint32_t k = 0;
        for (int64_t e : x) k += e > 0 ? 1u : 0u;
        return k;
    };
    for (size_t t = 0; t < nt; ++t)
        for (uint32_t j : tiles[t]) add(t, pm[j], 1);
    for (uint32_t iter = 0; iter < max_iter; ++iter) {
        size_t W = 0;
        uint32_t m = 0;
        for (size_t t = 0; t < nt; ++t)
            if (usize(cc[t]) > m) {
                m = usize(cc[t]);
                W = t;
            }
        uint32_t uw = 0;
        std::vector<uint32_t> cs;
        for (uint32_t c = 0; c < nu; ++c)
            if (cc[W][c] > 0) {
                uw |= 1u << c;
                cs.push_back(c);
            }
        std::stable_sort(cs.begin(), cs.end(),
                         [&](uint32_t a, uint32_t b) { return cc[W][a] < cc[W][b]; });
        bool done = false;
        for (uint32_t c : cs) {
            std::vector<uint32_t> A;
            for (uint32_t j : tiles[W])
                if (pm[j] >> c & 1u) A.push_back(j);
            struct Trade { uint32_t a; size_t B; uint32_t b; };
            std::vector<Trade> trades;
            std::set<uint32_t> used;
            bool all = true;
            for (uint32_t a : A) {
                bool hit = false;
                Trade tr{a, 0, 0};
                for (size_t B = 0; B < nt && !hit; ++B) {
                    if (B == W) continue;
                    for (uint32_t b : tiles[B]) {
                        if (used.count(b) || (pm[b] >> c & 1u) || (pm[b] & ~uw)) continue;
                        std::vector<int64_t> after = cc[B];
                        for (uint32_t q = 0; q < nu; ++q) {
                            if (pm[b] >> q & 1u) --after[q];
                            if (pm[a] >> q & 1u) ++after[q];
                        }
                        if (usize(after) + 1u <= m) {
                            tr.B = B;
                            tr.b = b;
                            hit = true;
                            break;
                        }
                    }
                }
                if (!hit) {
                    all = false;
                    break;
                }
                add(tr.B, pm[tr.b], -1);
                add(tr.B, pm[a], 1);
                add(W, pm[a], -1);
                add(W, pm[tr.b], 1);
                trades.push_back(tr);
                used.insert(tr.b);
            }
            if (all) {
                for (const Trade &tr : trades) {
                    auto &tw = tiles[W], &tb = tiles[tr.B];
                    tw.erase(std::find(tw.begin(), tw.end(), tr.a));
                    tw.push_back(tr.b);
                    tb.erase(std::find(tb.begin(), tb.end(), tr.b));
                    tb.push_back(tr.a);
                }
                done = true;
                break;
            }
            for (size_t k = trades.size(); k-- > 0;) {  // this cluster cannot go: undo
                const Trade &tr = trades[k];
                add(tr.B, pm[tr.b], 1);
                add(tr.B, pm[tr.a], -1);
                add(W, pm[tr.a], 1);
                add(W, pm[tr.b], -1);
            }
        }
        if (!done) break;
    }
    for (auto &t : tiles) std::sort(t.begin(), t.end());
    return tiles;
}

class K44WaveGraphCompiler {
  private:
    struct Shape3D {
        uint32_t c, h, w;
        bool is_1d;
    };
    struct PhysAlloc {
        uint32_t res_key;
        uint32_t num_ch;
        uint64_t canvas_off;
    };
    using ChanMap = std::map<std::string, std::vector<uint64_t>>;
    std::map<size_t, uint64_t> state_offs;  // TokenShift node -> state block offset

    static uint32_t make_res_key(uint32_t h, uint32_t w, bool is_1d) {
        if (is_1d) return 0x80000000u | w;
        return h == w ? h : ((h << 14) ^ w);
    }
    static uint64_t round_up(uint64_t v, uint64_t a) { return (v + a - 1u) / a * a; }

    static void init_node_bias(K44IRNode &n, uint32_t cout, const float *b) {
        n.bias_f32.assign(cout, 0.0f);
        n.bias_f16.assign(cout, 0u);
        if (!b) return;
        for (uint32_t i = 0; i < cout; ++i) {
            n.bias_f32[i] = b[i];
            n.bias_f16[i] = float_to_half(b[i]);
        }
    }

    static K44ExecCmd make_base_cmd(const K44IRNode &n, K44CmdType t, uint32_t rkey_in,
                                    uint32_t rkey_out, uint64_t src_off, uint64_t dst_off) {
        K44ExecCmd c{};
        c.name = n.name;
        c.type = t;
        c.Cin = n.cin ? n.cin : n.cout;
        c.Cout = c.logical_Cout = n.cout;
        c.h_in = n.h_in;
        c.w_in = n.w_in;
        c.h_out = n.h_out;
        c.w_out = n.w_out;
        c.res_key_in = rkey_in;
        c.res_key_out = rkey_out;
        c.src_off = src_off;
        c.y_off = dst_off;
        return c;
    }

    static uint32_t sparse_cout_pad(const K44IRNode &n) {
        return (uint32_t)round_up(n.cout, std::lcm<uint64_t>(16u, std::max(1u, n.cluster)));
    }

    // ---------------------------------------------------------------------------------------
    // Pass 1: shapes ([C, H, W] 2-D, [D, 1, tokens] 1-D) and zero-copy view bookkeeping.
    // ---------------------------------------------------------------------------------------
    void pass1_infer_shapes(K44WavePlan &plan, std::map<std::string, Shape3D> &shapes) {
        if (!nodes.empty() && nodes[0].op_type == "Input" && nodes[0].is_1d_tokens &&
            opts.batch_size > 1u && nodes[0].w_out == 1u)
            nodes[0].w_in = nodes[0].w_out = opts.batch_size;
        std::vector<K44IRNode> out;
        out.reserve(nodes.size() + 8u);
        for (auto &n : nodes) {
            const std::string &op = n.op_type;
            auto in_shape = [&](size_t i = 0) -> Shape3D {
                auto it = shapes.find(n.in_tensors.at(i));
                if (it == shapes.end())
                    throw std::runtime_error("node '" + n.name + "': unknown input tensor '" +
                                             n.in_tensors[i] + "'");
                return it->second;
            };
            if (op == "Input") {
                shapes[n.out_tensors[0]] = {n.cout, n.h_out, n.w_out, n.is_1d_tokens};
                plan.input_c = n.cout;
                plan.input_h = n.h_out;
                plan.input_w = n.w_out;
                // (the reference keys 2-D inputs by h alone, which names no layout when h != w)
                plan.input_res_key = make_res_key(n.h_out, n.w_out, n.is_1d_tokens);
            } else if (op == "Flatten") {
                const Shape3D s = in_shape();
                n.cin = s.c;
                n.cout = s.c * s.h * s.w;
                n.h_in = s.h;
                n.w_in = s.w;
                n.h_out = n.w_out = 1u;
                n.is_1d_tokens = true;
                shapes[n.out_tensors[0]] = {n.cout, 1u, 1u, true};
                plan.num_zero_copy_flattens++;
            } else if (op == "Split") {
                const Shape3D s = in_shape();
                n.is_1d_tokens = s.is_1d;
                for (const auto &o : n.out_tensors) shapes[o] = s;
                plan.num_eliminated_splits++;
            } else if (op == "Slice") {
                const Shape3D s = in_shape();
                n.is_1d_tokens = s.is_1d;
                for (size_t k = 0; k < n.out_tensors.size(); ++k) {
                    const uint32_t c = n.slice_sizes.empty()
                                           ? s.c / (uint32_t)n.out_tensors.size()
                                           : n.slice_sizes[k];
                    shapes[n.out_tensors[k]] = {c, s.h, s.w, s.is_1d};
                }
                plan.num_eliminated_splits++;
            } else if (op == "Concat") {
                const Shape3D s0 = in_shape();
                n.is_1d_tokens = s0.is_1d;
                uint32_t sum = 0;
                for (size_t i = 0; i < n.in_tensors.size(); ++i) sum += in_shape(i).c;
                shapes[n.out_tensors[0]] = {sum, s0.h, s0.w, s0.is_1d};
                plan.num_eliminated_concats++;
            } else if (op == "Convolution") {
                Shape3D s = in_shape();
                if (!s.is_1d && n.kh == 1u && n.kw == 1u && n.cin == s.c * s.h * s.w &&
                    n.cin != s.c) {
                    K44IRNode f;
                    f.op_type = "Flatten";
                    f.name = n.name + "_auto_flatten";
                    const std::string flat = n.in_tensors[0] + "_flat_view";
                    f.in_tensors = {n.in_tensors[0]};
                    f.out_tensors = {flat};
                    f.cin = s.c;
                    f.cout = s.c * s.h * s.w;
                    f.h_in = s.h;
                    f.w_in = s.w;
                    f.h_out = f.w_out = 1u;
                    f.is_1d_tokens = true;
                    out.push_back(std::move(f));
                    n.in_tensors[0] = flat;
                    s = {s.c * s.h * s.w, 1u, 1u, true};
                    shapes[flat] = s;
                    plan.num_zero_copy_flattens++;
                }
                n.is_1d_tokens = s.is_1d;
                n.h_in = s.h;
                n.w_in = s.w;
                n.h_out = s.is_1d ? 1u : s.h / n.stride;
                n.w_out = s.is_1d ? s.w : s.w / n.stride;
                shapes[n.out_tensors[0]] = {n.cout, n.h_out, n.w_out, s.is_1d};
            } else if (op == "SparseWave" || op == "PrunedWave") {
                const Shape3D s = in_shape();
                if (!s.is_1d)
                    throw std::runtime_error("sparse wave '" + n.name +
                                             "': input must be a 1-D token tensor");
                n.is_1d_tokens = true;
                n.cin = s.c;
                n.h_in = s.h;
                n.w_in = s.w;
                n.h_out = 1u;
                n.w_out = s.w;
                shapes[n.out_tensors[0]] = {n.cout, 1u, s.w, true};
            } else if (op == "TokenShift" || op == "ArgMax" || op == "Embedding") {
                const Shape3D s = in_shape();
                if (!s.is_1d)
                    throw std::runtime_error("node '" + n.name + "': needs a 1-D token tensor");
                n.is_1d_tokens = true;
                n.h_in = n.h_out = s.h;
                n.w_in = n.w_out = s.w;
                if (op == "TokenShift") {
                    n.cin = n.cout = s.c;
                    if (n.table.size() != (size_t)s.c * n.rf)
                        throw std::runtime_error("token shift '" + n.name +
                                                 "': mix table is not [channels][rf]");
                }
                if (op == "ArgMax") {
                    n.cin = s.c;
                    n.cout = 1u;
                }
                shapes[n.out_tensors[0]] = {n.cout, s.h, s.w, true};
            } else if (op == "Deconvolution") {
                const Shape3D s = in_shape();
                n.is_1d_tokens = false;
                n.h_in = s.h;
                n.w_in = s.w;
                n.h_out = s.h * n.stride;
                n.w_out = s.w * n.stride;
                shapes[n.out_tensors[0]] = {n.cout, n.h_out, n.w_out, false};
            } else if (op == "Pooling" || op == "Interp") {
                const Shape3D s = in_shape();
                n.cin = n.cout = s.c;
                n.h_in = s.h;
                n.w_in = s.w;
                n.h_out = op == "Pooling" ? s.h / n.stride : s.h * 2u;
                n.w_out = op == "Pooling" ? s.w / n.stride : s.w * 2u;
                shapes[n.out_tensors[0]] = {n.cout, n.h_out, n.w_out, false};
            } else if (op == "RMSNorm" || op == "SwiGLU" || op == "RoPEAttention") {
                const Shape3D s = in_shape();
                n.is_1d_tokens = s.is_1d;
                n.h_in = n.h_out = s.h;
                n.w_in = n.w_out = s.w;
                if (op == "SwiGLU") n.cin = n.cout = s.c;
                shapes[n.out_tensors[0]] =
                    op == "RoPEAttention" ? Shape3D{n.cout, s.h, s.w, s.is_1d} : s;
            }
            out.push_back(std::move(n));
        }
        nodes = std::move(out);
    }

    // ---------------------------------------------------------------------------------------
    // Pass 2: W[n][ch] *= gamma[ch] for every 1x1 consumer of an RMSNorm output, when every
    // consumer (through Split aliases) is a 1x1 projection and none uses it as a residual.
    // ---------------------------------------------------------------------------------------
    void pass2_fold_rmsnorm(K44WavePlan &plan) {
        if (!opts.fold_rmsnorm_gamma) return;
        for (size_t i = 0; i < nodes.size(); ++i) {
            K44IRNode &norm = nodes[i];
            if (norm.op_type != "RMSNorm") continue;
            if (norm.gamma_folded) {
                plan.num_folded_rmsnorms++;
                continue;
            }
            std::set<std::string> alias = {norm.out_tensors[0]};
            std::vector<size_t> users;
            bool foldable = true;
            for (size_t j = i + 1; j < nodes.size(); ++j) {
                const K44IRNode &u = nodes[j];
                if (u.op_type == "Split" && alias.count(u.in_tensors[0])) {
                    alias.insert(u.out_tensors.begin(), u.out_tensors.end());
                    continue;
                }
                for (const auto &t : u.in_tensors) {
                    if (!alias.count(t)) continue;
                    if (u.op_type == "Convolution" && u.kh == 1u && u.kw == 1u)
                        users.push_back(j);
                    else
                        foldable = false;
                }
                if (!u.residual_tensor.empty() && alias.count(u.residual_tensor)) foldable = false;
            }
            if (!foldable || users.empty()) continue;
            const std::vector<float> &g = norm.bias_f32;
            for (size_t j : users) {
                K44IRNode &u = nodes[j];
                const bool have_f32 = !u.weights_f32.empty();
                for (uint32_t r = 0; r < u.cout; ++r)
                    for (uint32_t ch = 0; ch < u.cin; ++ch) {
                        const size_t at = (size_t)r * u.cin + ch;
                        if (have_f32) {
                            u.weights_f32[at] *= g[ch];
                            u.weights_f16[at] = float_to_half(u.weights_f32[at]);
                        } else {
                            u.weights_f16[at] = float_to_half(half_to_float(u.weights_f16[at]) * g[ch]);
                        }
                    }
            }
            norm.gamma_folded = true;
            plan.num_folded_rmsnorms++;
        }
    }

    // ---------------------------------------------------------------------------------------
    // Pass 3: frames per wave, one resolution descriptor per distinct shape key, wave configs.
    // ---------------------------------------------------------------------------------------
    void pass3_build_layouts(K44WavePlan &plan, const std::map<std::string, Shape3D> &shapes,
                             std::vector<K44WaveConfig> &cfg) {
        const bool graph_1d = !nodes.empty() && nodes[0].op_type == "Input" &&
                              nodes[0].is_1d_tokens;
        const bool tok64 = !graph_1d && opts.batch_size >= 64u && opts.batch_size % 64u == 0u;
        uint32_t frames = graph_1d ? 1u : (tok64 ? 64u : std::min(std::max(1u, opts.batch_size), 8u));
        if (tok64) {
            const char *env = std::getenv("WAVEC_WAVE_BATCH");
            const int wb = env ? std::atoi(env) : 0;
            if (wb >= 64 && wb % 64 == 0)
                frames = std::min(opts.batch_size, (uint32_t)wb);
            else if (opts.reuse_canvas && opts.batch_size <= 256u)
                frames = opts.batch_size;
        }
        plan.batch_size = std::max(1u, opts.batch_size);
        plan.wave_batch_size = frames;
        plan.is_image_token64 = tok64;
        for (const auto &kv : shapes) {
            const uint32_t key = make_res_key(kv.second.h, kv.second.w, kv.second.is_1d);
            if (!plan.res_map.count(key))
                plan.res_map[key].init(kv.second.h, kv.second.w, kv.second.is_1d, frames);
        }
        plan.hw_profile = opts.hw_profile;
        const uint32_t img_blocks = tok64 ? frames / 64u : 1u;
        cfg.assign(nodes.size(), K44WaveConfig{16u, 16u, 0u, 0u, 1u});
        for (size_t i = 0; i < nodes.size(); ++i) {
            const K44IRNode &n = nodes[i];
            if (n.op_type == "Convolution") {
                auto extent = [&](uint32_t h, uint32_t w) -> uint32_t {
                    if (n.is_1d_tokens)
                        return std::max(1u, plan.res_map.at(make_res_key(h, w, true)).num_tiles);
                    return std::max(1u, h * w) * img_blocks;
                };
                cfg[i] = select_optimal_wave_config(n.cin, n.cout, n.kh, n.kw,
                                                    extent(n.h_in, n.w_in),
                                                    extent(n.h_out, n.w_out),
                                                    opts.force_cluster_size, opts.hw_profile,
                                                    opts.max_B_per_wave);
            } else if (n.op_type == "SparseWave") {
                cfg[i] = K44WaveConfig{std::max(1u, n.cluster), sparse_cout_pad(n), 0u, 0u, 1u};
            }
        }
    }

    // ---------------------------------------------------------------------------------------
    // Pass 4: allocation ids (views share their source's ids), last use, best-fit placement on
    // a 64-element grid with coalescing of freed neighbours, then scratch regions (S2D,
    // up-conv quadrants), KV cache, attention probabilities; canvas rounded up to 128.
    // ---------------------------------------------------------------------------------------
    void pass4_allocate_canvas(K44WavePlan &plan, const std::vector<K44WaveConfig> &cfg,
                               std::map<int, PhysAlloc> &allocs, std::vector<int> &out_aid,
                               std::map<uint32_t, uint64_t> &s2d_base,
                               std::map<uint32_t, uint64_t> &quad_base,
                               std::map<size_t, std::pair<uint64_t, uint64_t>> &kv_offs,
                               uint64_t &probs_off) {
        state_offs.clear();
        std::map<std::string, std::set<int>> ids;
        out_aid.assign(nodes.size(), -1);
        int next_id = 0;
        for (size_t i = 0; i < nodes.size(); ++i) {
            const K44IRNode &n = nodes[i];
            if (n.op_type == "Split" || n.op_type == "Slice" || n.op_type == "Flatten") {
                const std::set<int> src = ids.at(n.in_tensors[0]);
                for (const auto &o : n.out_tensors) ids[o] = src;
            } else if (n.op_type == "Concat") {
                std::set<int> u;
                for (const auto &t : n.in_tensors) {
                    const auto &s = ids.at(t);
                    u.insert(s.begin(), s.end());
                }
                ids[n.out_tensors[0]] = u;
            } else {
                const int id = next_id++;
                const uint32_t ch = (n.op_type == "Convolution" || n.op_type == "SparseWave")
                                        ? cfg[i].total_cout_pad()
                                        : n.cout;  // PrunedWave: mapped stores, no padding
                allocs[id] = {make_res_key(n.h_out, n.w_out, n.is_1d_tokens), ch, 0u};
                ids[n.out_tensors[0]] = {id};
                out_aid[i] = id;
            }
        }

        std::map<int, size_t> last;
        last[0] = nodes.size();
        if (ids.count(default_output_tensor))
            for (int id : ids.at(default_output_tensor)) last[id] = nodes.size();
        for (size_t i = 0; i < nodes.size(); ++i) {
            auto touch = [&](const std::string &t) {
                auto it = ids.find(t);
                if (it == ids.end()) return;
                for (int id : it->second) last[id] = std::max(last[id], i);
            };
            for (const auto &t : nodes[i].in_tensors) touch(t);
            if (!nodes[i].residual_tensor.empty()) touch(nodes[i].residual_tensor);
        }

        plan.reuse_canvas = opts.reuse_canvas;
        std::map<uint32_t, uint32_t> s2d_ch, quad_ch;
        uint64_t subwave_peak = 0u;
        for (size_t i = 0; i < nodes.size(); ++i) {
            const K44IRNode &n = nodes[i];
            if (n.op_type == "Convolution" && n.stride == 2u) {
                if (!plan.is_image_token64) {
                    uint32_t &v = s2d_ch[make_res_key(n.h_out, n.w_out, false)];
                    v = std::max(v, 4u * n.cin);
                } else if (cfg[i].num_sub_b > 1u) {
                    subwave_peak = std::max<uint64_t>(
                        subwave_peak, (uint64_t)cfg[i].total_cout_pad() *
                                          plan.res_map.at(make_res_key(n.h_in, n.w_in, false))
                                              .channel_stride);
                }
            } else if (n.op_type == "Deconvolution") {
                uint32_t &v = quad_ch[make_res_key(n.h_in, n.w_in, false)];
                v = std::max(v, 4u * round_up_16(n.cout));
            }
        }

        struct Interval {
            uint64_t start, len;
        };
        std::vector<Interval> free_list;  // kept sorted by start
        uint64_t peak = 0u;
        std::map<int, Interval> placed;
        std::set<int> live;
        for (size_t i = 0; i < nodes.size(); ++i) {
            const int id = out_aid[i];
            if (id != -1) {
                const uint64_t need =
                    round_up((uint64_t)allocs[id].num_ch *
                                 plan.res_map.at(allocs[id].res_key).channel_stride,
                             64u);
                int best = -1;
                for (size_t k = 0; k < free_list.size(); ++k)
                    if (free_list[k].len >= need &&
                        (best < 0 || free_list[k].len < free_list[(size_t)best].len))
                        best = (int)k;
                uint64_t at;
                if (best >= 0) {
                    Interval &f = free_list[(size_t)best];
                    at = f.start;
                    if (f.len == need) {
                        free_list.erase(free_list.begin() + best);
                    } else {
                        f.start += need;
                        f.len -= need;
                    }
                } else if (!free_list.empty() &&
                           free_list.back().start + free_list.back().len == peak) {
                    at = free_list.back().start;
                    free_list.pop_back();
                    peak = at + need;
                } else {
                    at = peak;
                    peak += need;
                }
                placed[id] = {at, need};
                allocs[id].canvas_off = at;
                live.insert(id);
            }
            bool freed = false;
            for (auto it = live.begin(); it != live.end();) {
                if (last[*it] <= i) {
                    free_list.push_back(placed[*it]);
                    it = live.erase(it);
                    freed = true;
                } else {
                    ++it;
                }
            }
            if (freed && free_list.size() > 1u) {
                std::sort(free_list.begin(), free_list.end(),
                          [](const Interval &a, const Interval &b) { return a.start < b.start; });
                std::vector<Interval> merged;
                for (const Interval &f : free_list) {
                    if (!merged.empty() && merged.back().start + merged.back().len == f.start)
                        merged.back().len += f.len;
                    else
                        merged.push_back(f);
                }
                free_list.swap(merged);
            }
        }

        uint64_t cur = round_up(peak, 64u);
        uint64_t s2d_max = 0u;
        for (const auto &kv : s2d_ch) {
            s2d_base[kv.first] = cur;
            s2d_max = std::max<uint64_t>(s2d_max, (uint64_t)kv.second *
                                                      plan.res_map.at(kv.first).channel_stride);
        }
        cur += round_up(s2d_max, 64u);
        uint64_t quad_max = subwave_peak;
        for (const auto &kv : quad_ch) {
            quad_base[kv.first] = cur;
            quad_max = std::max<uint64_t>(quad_max, (uint64_t)kv.second *
                                                        plan.res_map.at(kv.first).channel_stride);
        }
        cur += round_up(quad_max, 64u);

        probs_off = 0u;
        uint64_t kv_total = 0u;
        if (opts.kv_cache_max_seq > 0u) {
            uint32_t max_hq = 0u;
            for (size_t i = 0; i < nodes.size(); ++i) {
                const K44IRNode &n = nodes[i];
                if (n.op_type != "RoPEAttention") continue;
                const uint64_t kv = (uint64_t)n.h_kv * n.head_dim * opts.kv_cache_max_seq;
                kv_offs[i] = {cur, cur + kv};
                cur += 2u * kv;
                kv_total += 2u * kv;
                max_hq = std::max(max_hq, n.h_q);
            }
            if (max_hq > 0u) {
                probs_off = cur;
                cur += (uint64_t)max_hq * opts.kv_cache_max_seq;
            }
        }
        // Token-shift state blocks (build extension): [C][rf-1][64] per TokenShift node.
        for (size_t i = 0; i < nodes.size(); ++i) {
            const K44IRNode &n = nodes[i];
            if (n.op_type != "TokenShift" || n.rf < 2u) continue;
            state_offs[i] = cur;
            cur += round_up((uint64_t)n.cout * (n.rf - 1u) * 64u, 64u);
        }
        cur = round_up(cur, 128u);
        plan.kv_cache_elems = kv_total;
        plan.canvas_elems = cur ? cur : 128u;
        plan.input_off = allocs.empty() ? 0u : allocs[0].canvas_off;
    }

    void reserve_residual(K44WavePlan &plan, uint64_t res_off, uint32_t cout_pad,
                          uint32_t out_stride) {
        const uint64_t end = res_off + (uint64_t)cout_pad * out_stride;
        if (end > plan.canvas_elems) plan.canvas_elems = round_up(end, 128u);
    }

    // tap_offset(base, dy, dx) - base, evaluated with 64-bit bases (dy, dx >= -1).
    static uint64_t tap_rel(const K44ResDesc &L, int dy, int dx) {
        if (L.is_1d_tokens) return (uint64_t)(int64_t)dx;
        const uint64_t rel = (uint64_t)(1 + dy) * L.W_pad + (uint64_t)(1 + dx);
        return L.is_image_token64 ? rel * 64u : rel;
    }

    static uint32_t idx_word(uint64_t v, const std::string &who) {
        if (v > 0xffffffffULL)
            throw std::runtime_error("wave '" + who +
                                     "': gather offset exceeds the 32-bit index range");
        return (uint32_t)v;
    }

    // 2x2 stride-2 transposed convolution = 1x1 wave into a quadrant scratch + scatter command.
    void emit_deconv_waves(K44IRNode &n, uint32_t rkey_in, uint32_t rkey_out, uint64_t dst_off,
                           uint64_t quad_off, const std::vector<uint64_t> &in_chs,
                           K44WavePlan &plan) {
        const K44ResDesc &L = plan.res_map.at(rkey_in);
        const uint32_t cout_al = round_up_16(n.cout), cout_q = 4u * cout_al;
        const uint32_t tiles = L.is_image_token64 ? (L.H * (L.W + 4u) + 63u) / 64u
                                                  : L.tiles_per_frame;
        const uint32_t cl = choose_cluster_size(cout_q, tiles, opts.force_cluster_size);
        const uint32_t B = round_up_32(n.cin);
        std::vector<uint32_t> idx((size_t)(cout_q / cl) * B, 0u);
        for (uint32_t r = 0; r < cout_q / cl; ++r)
            for (uint32_t ch = 0; ch < n.cin; ++ch)
                idx[(size_t)r * B + ch] = idx_word(in_chs[ch] + tap_rel(L, 0, 0), n.name);
        std::vector<uint16_t> w, bias(cout_q, 0u);
        if (!n.weights_f16.empty()) {
            w.assign((size_t)cout_q * B, 0u);
            for (uint32_t q = 0; q < 4u; ++q)
                for (uint32_t j = 0; j < n.cout; ++j) {
                    const uint32_t row = q * cout_al + j;
                    if (j < n.bias_f16.size()) bias[row] = n.bias_f16[j];
                    for (uint32_t ch = 0; ch < n.cin; ++ch)
                        w[(size_t)row * B + ch] = n.weights_f16[((size_t)j * n.cin + ch) * 4u + q];
                }
        }
        K44ExecCmd c = make_base_cmd(n, K44CmdType::K44_WAVE, rkey_in, rkey_in, 0u, quad_off);
        c.Cout = cout_q;
        c.logical_Cout = 4u * n.cout;
        c.cluster_size = cl;
        c.B = B;
        c.B_raw = n.cin;
        c.B_vec16 = B / 16u;
        c.has_bias = true;
        c.act = K44Act::NONE;
        c.has_residual = false;
        c.h_out = n.h_in;
        c.w_out = n.w_in;
        const double sf = 2.0 * n.cin * (double)cout_q * (double)(n.h_in * n.w_in) / 1e9;
        c.gflops = (double)plan.wave_batch_size * sf;
        plan.single_frame_gflops += sf;
        plan.total_gflops += c.gflops;
        pack_wave_buffers(c, w, idx, bias, plan);
        plan.cmds.push_back(std::move(c));
        plan.num_wave_dispatches++;
        K44ExecCmd s =
            make_base_cmd(n, K44CmdType::SCATTER_UP2X2, rkey_in, rkey_out, quad_off, dst_off);
        s.name = n.name + "_scatter2x2";
        s.Cin = cout_q;
        plan.cmds.push_back(std::move(s));
    }

    // Dense 1-D / 2-D convolution (incl. 1x1 linear): every index row lists all input channels
    // x taps (syn = ch * taps + ky * kw + kx); stride-2 2-D convs read a polyphase S2D scratch.
    void emit_conv_waves(K44IRNode &n, const K44WaveConfig &wc, uint32_t rkey_in,
                         uint32_t rkey_out, uint64_t dst_off,
                         const std::map<uint32_t, uint64_t> &s2d_base, const ChanMap &chan,
                         K44WavePlan &plan) {
        const K44ResDesc &Li = plan.res_map.at(rkey_in);
        const K44ResDesc &Lo = plan.res_map.at(rkey_out);
        const bool tok64 = plan.is_image_token64;
        const uint32_t cout_pad = wc.total_cout_pad();
        const std::vector<uint64_t> &in_chs = chan.at(n.in_tensors[0]);
        const bool has_res = !n.residual_tensor.empty();
        const uint64_t res_off = has_res ? chan.at(n.residual_tensor)[0] : 0u;
        if (has_res) reserve_residual(plan, res_off, cout_pad, Lo.channel_stride);
        const uint32_t taps = n.kh * n.kw, b_raw = taps * n.cin;
        const bool polyphase = n.stride == 2u && !tok64;
        uint64_t s2d_off = 0u;
        if (polyphase) {
            s2d_off = s2d_base.at(rkey_out);
            K44ExecCmd s = make_base_cmd(n, K44CmdType::S2D_2X2, rkey_in, rkey_out, in_chs[0],
                                         s2d_off);
            s.name = n.name + "_s2d_2x2";
            s.Cout = s.logical_Cout = 4u * n.cin;
            plan.cmds.push_back(std::move(s));
        }
        auto tap = [&](uint32_t ch, uint32_t ky, uint32_t kx) -> uint64_t {
            if (polyphase) {
                const uint32_t py = ky == 1u ? 0u : 1u, px = kx == 1u ? 0u : 1u;
                const uint64_t poly = s2d_off + (uint64_t)(4u * ch + 2u * py + px) * Lo.channel_stride;
                return poly + tap_rel(Lo, ky == 0u ? -1 : 0, kx == 0u ? -1 : 0);
            }
            if (n.kh == 1u && n.kw == 1u) return in_chs[ch] + tap_rel(Lo, 0, 0);
            const int dy = (int)ky - (int)(n.kh / 2u), dx = (int)kx - (int)(n.kw / 2u);
            return in_chs[ch] + tap_rel(n.stride == 2u ? Li : Lo, dy, dx);
        };
        const uint32_t B = round_up_32(b_raw);
        const uint32_t S = wc.S1, rows = wc.Cout_pad1 / S;
        const uint32_t cout_log = std::min(wc.Cout_pad1, n.cout);
        std::vector<uint32_t> idx((size_t)rows * B, 0u);
        for (uint32_t r = 0; r < rows; ++r)
            for (uint32_t ch = 0; ch < n.cin; ++ch)
                for (uint32_t ky = 0; ky < n.kh; ++ky)
                    for (uint32_t kx = 0; kx < n.kw; ++kx)
                        idx[(size_t)r * B + ch * taps + ky * n.kw + kx] =
                            idx_word(tap(ch, ky, kx), n.name);
        std::vector<uint16_t> bias(wc.Cout_pad1, 0u);
        for (uint32_t j = 0; j < cout_log && j < n.bias_f16.size(); ++j) bias[j] = n.bias_f16[j];
        std::vector<uint16_t> w;
        if (!n.weights_f16.empty()) {
            w.assign((size_t)wc.Cout_pad1 * B, 0u);
            for (uint32_t j = 0; j < cout_log; ++j)
                std::memcpy(&w[(size_t)j * B], &n.weights_f16[(size_t)j * b_raw], b_raw * 2u);
        }
        K44ExecCmd c = make_base_cmd(n, K44CmdType::K44_WAVE,
                                     (n.stride == 2u && tok64) ? rkey_in : rkey_out, rkey_out,
                                     polyphase ? s2d_off : in_chs[0], dst_off);
        c.Cout = wc.Cout_pad1;
        c.logical_Cout = cout_log;
        c.cluster_size = S;
        c.B = B;
        c.B_raw = b_raw;
        c.B_vec16 = B / 16u;
        c.has_bias = true;
        c.act = n.act;
        c.has_residual = has_res;
        c.res_off = has_res ? res_off : 0u;
        c.seg_len = (n.kh == 1u && n.kw == 1u) ? n.cin : 1u;
        const double sf =
            2.0 * n.cin * (double)cout_log * taps * (double)(n.h_out * n.w_out) / 1e9;
        c.gflops = (double)plan.wave_batch_size * sf;
        plan.single_frame_gflops += sf;
        plan.total_gflops += c.gflops;
        pack_wave_buffers(c, w, idx, bias, plan);
        plan.cmds.push_back(std::move(c));
        plan.num_wave_dispatches++;
    }

    // One K44_WAVE over explicit index rows (build extension): `cout` neurons, neurons
    // [r*cluster, (r+1)*cluster) share row r, which lists the input channel of each of the fan_in
    // synapses.  Canvas offsets come from the input tensor's channel offset list, so views
    // (Concat / Slice) work as they do for dense waves.  cmap (optional, one entry per neuron)
    // sends neuron j to output channel cmap[j]; 0xFFFF marks an empty slot that stores nothing.
    struct SparseRows {
        std::string name;
        uint32_t cout, fan_in, cluster, seg_len;
        const uint32_t *rows;   // [cout/cluster][fan_in]
        const uint16_t *w;      // [cout][fan_in]
        const uint16_t *bias;   // [cout] or nullptr
        std::vector<uint16_t> cmap;
        uint64_t nnz;           // real synapses (effective FLOPs = 2 nnz tokens)
    };

    void emit_sparse_rows(const K44IRNode &n, const SparseRows &sr, uint32_t rkey_in,
                          uint32_t rkey_out, uint64_t dst_off, const ChanMap &chan,
                          K44WavePlan &plan) {
        const K44ResDesc &Lo = plan.res_map.at(rkey_out);
        const std::vector<uint64_t> &in_chs = chan.at(n.in_tensors[0]);
        const bool has_res = !n.residual_tensor.empty();
        const uint64_t res_off = has_res ? chan.at(n.residual_tensor)[0] : 0u;
        const uint32_t cl = std::max(1u, sr.cluster);
        const uint32_t cout_pad =
            (uint32_t)round_up(sr.cout, std::lcm<uint64_t>(16u, cl));
        const bool mapped = !sr.cmap.empty();
        if (has_res && !mapped) reserve_residual(plan, res_off, cout_pad, Lo.channel_stride);
        const uint32_t b_raw = sr.fan_in, B = round_up_32(b_raw);
        const uint32_t rows_real = sr.cout / cl, rows = cout_pad / cl;
        uint64_t hi_off = 0u;
        for (size_t i = 0; i < (size_t)rows_real * b_raw; ++i) {
            const uint32_t p = sr.rows[i];
            if (p >= in_chs.size())
                throw std::runtime_error("sparse wave '" + sr.name +
                                         "': synapse position beyond the input channel count");
            hi_off = std::max(hi_off, in_chs[p]);
        }
        const bool row_mode = hi_off > 0xffffffffULL;
        uint64_t stride = plan.res_map.at(rkey_in).channel_stride;
        if (row_mode) {
            for (size_t c = 0; c < in_chs.size(); ++c)
                if (in_chs[c] != in_chs[0] + c * stride)
                    throw std::runtime_error(
                        "sparse wave '" + sr.name +
                        "': input beyond 2^32 canvas elements must be one contiguous tensor");
        }
        std::vector<uint32_t> idx((size_t)rows * B, 0u);
        for (uint32_t r = 0; r < rows_real; ++r)
            for (uint32_t s = 0; s < b_raw; ++s) {
                const uint32_t p = sr.rows[(size_t)r * b_raw + s];
                idx[(size_t)r * B + s] = row_mode ? p : (uint32_t)in_chs[p];
            }
        std::vector<uint16_t> w((size_t)cout_pad * B, 0u), bias(cout_pad, 0u);
        for (uint32_t j = 0; j < sr.cout; ++j) {
            std::memcpy(&w[(size_t)j * B], &sr.w[(size_t)j * b_raw], b_raw * 2u);
            if (sr.bias) bias[j] = sr.bias[j];
        }
        std::vector<uint16_t> cmap;
        if (mapped) {
            cmap = sr.cmap;
            cmap.resize(cout_pad, 0xffffu);
        }
        K44ExecCmd c =
            make_base_cmd(n, K44CmdType::K44_WAVE, rkey_in, rkey_out, in_chs[0], dst_off);
        c.name = sr.name;
        c.Cout = cout_pad;
        c.logical_Cout = mapped ? n.cout : sr.cout;
        c.cluster_size = cl;
        c.B = B;
        c.B_raw = b_raw;
        c.B_vec16 = B / 16u;
        c.has_bias = true;
        c.act = n.act;
        c.has_residual = has_res;
        c.res_off = has_res ? res_off : 0u;
        c.seg_len = sr.seg_len;
        c.idx_mode = row_mode ? 1u : 0u;
        c.idx_stride = row_mode ? stride : 1u;
        const double sf = 2.0 * (double)sr.nnz * (double)(n.h_out * n.w_out) / 1e9;
        c.gflops = (double)plan.wave_batch_size * sf;
        plan.single_frame_gflops += sf;
        plan.total_gflops += c.gflops;
        pack_wave_buffers(c, w, idx, bias, plan, cmap);
        if (row_mode) c.x_base_off = in_chs[0];
        plan.cmds.push_back(std::move(c));
        plan.num_wave_dispatches++;
    }

    void emit_sparse_wave(K44IRNode &n, uint32_t rkey_in, uint32_t rkey_out, uint64_t dst_off,
                          const ChanMap &chan, K44WavePlan &plan) {
        SparseRows sr{n.name,        n.cout,
                      n.fan_in,      std::max(1u, n.cluster),
                      n.seg_len,     n.rows.data(),
                      n.weights_f16.data(), n.bias_f16.empty() ? nullptr : n.bias_f16.data(),
                      {},            (uint64_t)n.cout * n.fan_in};
        emit_sparse_rows(n, sr, rkey_in, rkey_out, dst_off, chan, plan);
    }

    // Pattern-sorted pruned projection: one K44_WAVE per sub-wave, all writing the node's output
    // tensor through their cout_map.
    void emit_pruned_wave(K44IRNode &n, uint32_t rkey_in, uint32_t rkey_out, uint64_t dst_off,
                          const ChanMap &chan, K44WavePlan &plan) {
        const uint32_t tile = n.cluster, S = n.seg_len;
        size_t row_at = 0, slot_at = 0;
        std::vector<uint32_t> rows;
        for (size_t p = 0; p < n.part_tiles.size(); ++p) {
            const uint32_t tiles = n.part_tiles[p], K = n.part_k[p], fan = K * S;
            rows.assign((size_t)tiles * fan, 0u);
            for (uint32_t t = 0; t < tiles; ++t)
                for (uint32_t k = 0; k < K; ++k)
                    for (uint32_t s = 0; s < S; ++s)
                        rows[((size_t)t * K + k) * S + s] = n.rows[row_at + (size_t)t * K + k] + s;
            const uint32_t slots = tiles * tile;
            uint64_t real = 0;
            for (uint32_t j = 0; j < slots; ++j) real += n.cout_map[slot_at + j] != 0xffffu;
            SparseRows sr{n.part_tiles.size() > 1u ? n.name + "/" + std::to_string(p) : n.name,
                          slots,
                          fan,
                          tile,
                          S,
                          rows.data(),
                          n.weights_f16.data() + n_weights_before(n, p),
                          n.bias_f16.data() + slot_at,
                          std::vector<uint16_t>(n.cout_map.begin() + slot_at,
                                                n.cout_map.begin() + slot_at + slots),
                          real * (n.nnz / std::max<uint32_t>(1u, n.cout))};
            emit_sparse_rows(n, sr, rkey_in, rkey_out, dst_off, chan, plan);
            row_at += (size_t)tiles * K;
            slot_at += slots;
        }
    }

    static size_t n_weights_before(const K44IRNode &n, size_t part) {
        size_t at = 0;
        for (size_t p = 0; p < part; ++p)
            at += (size_t)n.part_tiles[p] * n.cluster * n.part_k[p] * n.seg_len;
        return at;
    }

    // ---------------------------------------------------------------------------------------
    // Pass 5: channel offset lists (views are free), command stream, plan output descriptor.
    // ---------------------------------------------------------------------------------------
    void pass5_emit_commands(K44WavePlan &plan, const std::map<std::string, Shape3D> &shapes,
                             const std::vector<K44WaveConfig> &cfg,
                             const std::map<int, PhysAlloc> &allocs,
                             const std::vector<int> &out_aid,
                             const std::map<uint32_t, uint64_t> &s2d_base,
                             const std::map<uint32_t, uint64_t> &quad_base,
                             const std::map<size_t, std::pair<uint64_t, uint64_t>> &kv_offs,
                             uint64_t probs_off) {
        ChanMap chan;
        auto place = [&](const K44IRNode &n, int id, uint32_t nch) -> uint64_t {
            const PhysAlloc &a = allocs.at(id);
            const uint64_t st = plan.res_map.at(a.res_key).channel_stride;
            std::vector<uint64_t> v(nch);
            for (uint32_t c = 0; c < nch; ++c) v[c] = a.canvas_off + c * st;
            chan[n.out_tensors[0]] = std::move(v);
            return a.canvas_off;
        };
        for (size_t i = 0; i < nodes.size(); ++i) {
            K44IRNode &n = nodes[i];
            const std::string &op = n.op_type;
            const int id = out_aid[i];
            if (op == "Input") {
                place(n, id, n.cout);
            } else if (op == "Flatten") {
                const Shape3D s = shapes.at(n.in_tensors[0]);
                const K44ResDesc &L = plan.res_map.at(make_res_key(s.h, s.w, s.is_1d));
                const std::vector<uint64_t> &src = chan.at(n.in_tensors[0]);
                std::vector<uint64_t> v;
                v.reserve((size_t)s.c * s.h * s.w);
                for (uint32_t c = 0; c < s.c; ++c)
                    for (uint32_t y = 0; y < s.h; ++y)
                        for (uint32_t x = 0; x < s.w; ++x)
                            v.push_back(s.is_1d ? src[c] + x
                                                : src[c] + (uint64_t)(y + 1u) * L.W_pad + 4u + x);
                chan[n.out_tensors[0]] = std::move(v);
            } else if (op == "Split") {
                for (const auto &o : n.out_tensors) chan[o] = chan.at(n.in_tensors[0]);
            } else if (op == "Slice") {
                const std::vector<uint64_t> src = chan.at(n.in_tensors[0]);
                size_t at = 0;
                for (size_t k = 0; k < n.out_tensors.size(); ++k) {
                    const size_t len = n.slice_sizes.empty() ? src.size() / n.out_tensors.size()
                                                             : n.slice_sizes[k];
                    chan[n.out_tensors[k]] =
                        std::vector<uint64_t>(src.begin() + at, src.begin() + at + len);
                    at += len;
                }
            } else if (op == "Concat") {
                std::vector<uint64_t> cat;
                for (const auto &t : n.in_tensors) {
                    const auto &s = chan.at(t);
                    cat.insert(cat.end(), s.begin(), s.end());
                }
                chan[n.out_tensors[0]] = std::move(cat);
            } else if (op == "Pooling" || op == "Interp") {
                const uint32_t rk_in = make_res_key(n.h_in, n.w_in, false);
                const uint32_t rk_out = allocs.at(id).res_key;
                const uint64_t dst = place(n, id, n.cout);
                const K44CmdType t = op == "Interp" ? K44CmdType::UPSAMPLE_2X
                                                    : (n.kh == 2u ? K44CmdType::MAXPOOL_2X2
                                                                  : K44CmdType::MAXPOOL_5X5);
                plan.cmds.push_back(make_base_cmd(n, t, rk_in, rk_out,
                                                  chan.at(n.in_tensors[0])[0], dst));
            } else if (op == "RMSNorm") {
                const uint32_t rk = allocs.at(id).res_key;
                const uint64_t dst = place(n, id, n.cout);
                K44ExecCmd c = make_base_cmd(n, K44CmdType::RMSNORM_1D, rk, rk,
                                             chan.at(n.in_tensors[0])[0], dst);
                c.eps = n.eps;
                c.gamma_folded = n.gamma_folded;
                if (!n.gamma_folded) c.h_bias = n.bias_f16;
                plan.cmds.push_back(std::move(c));
            } else if (op == "SwiGLU") {
                const uint32_t rk = allocs.at(id).res_key;
                const uint64_t dst = place(n, id, n.cout);
                K44ExecCmd c = make_base_cmd(n, K44CmdType::SWIGLU_MUL_1D, rk, rk,
                                             chan.at(n.in_tensors[0])[0], dst);
                c.src2_off = chan.at(n.in_tensors[1])[0];
                plan.cmds.push_back(std::move(c));
            } else if (op == "RoPEAttention") {
                const uint32_t rk = allocs.at(id).res_key;
                const uint64_t dst = place(n, id, n.cout);
                K44ExecCmd c = make_base_cmd(n, K44CmdType::ROPE_GQA_ATTN_1D, rk, rk,
                                             chan.at(n.in_tensors[0])[0], dst);
                c.Cin = n.cout;
                c.h_q = n.h_q;
                c.h_kv = n.h_kv;
                c.head_dim = n.head_dim;
                c.rope_theta = n.rope_theta;
                c.llama3_rope_scaling = n.llama3_rope_scaling;
                c.src2_off = chan.at(n.in_tensors[1])[0];
                c.src3_off = chan.at(n.in_tensors[2])[0];
                if (opts.kv_cache_max_seq > 0u) {
                    c.kv_k_off = kv_offs.at(i).first;
                    c.kv_v_off = kv_offs.at(i).second;
                    c.kv_max_seq = opts.kv_cache_max_seq;
                    c.attn_probs_off = probs_off;
                }
                const double sf = 2.0 * n.cout * (double)n.w_out * (double)(n.w_out + 1u) / 1e9;
                c.gflops = (double)plan.wave_batch_size * sf;
                plan.single_frame_gflops += sf;
                plan.total_gflops += c.gflops;
                plan.cmds.push_back(std::move(c));
            } else if (op == "TokenShift" || op == "Embedding" || op == "ArgMax") {
                const uint32_t rk = allocs.at(id).res_key;
                const uint64_t dst = place(n, id, n.cout);
                const std::vector<uint64_t> &src = chan.at(n.in_tensors[0]);
                const uint64_t st = plan.res_map.at(rk).channel_stride;
                for (size_t c = 0; c < src.size(); ++c)
                    if (src[c] != src[0] + c * st)
                        throw std::runtime_error("node '" + n.name +
                                                 "': input channels must be one contiguous tensor");
                const K44CmdType t = op == "TokenShift" ? K44CmdType::TOKEN_SHIFT_1D
                                     : op == "Embedding" ? K44CmdType::EMBED_1D
                                                         : K44CmdType::ARGMAX_1D;
                K44ExecCmd c = make_base_cmd(n, t, rk, rk, src[0], dst);
                c.rf = n.rf;
                c.seq_len = n.seq_len;
                c.decode_state = n.decode_state;
                c.h_table = n.table;
                if (op == "Embedding") c.Cin = n.vocab;
                if (op == "ArgMax") c.Cin = n.cin;
                auto so = state_offs.find(i);
                if (so != state_offs.end()) c.state_off = so->second;
                plan.cmds.push_back(std::move(c));
            } else if (op == "Deconvolution") {
                const uint32_t rk_in = make_res_key(n.h_in, n.w_in, false);
                const uint32_t rk_out = allocs.at(id).res_key;
                const uint64_t dst = place(n, id, n.cout);
                emit_deconv_waves(n, rk_in, rk_out, dst, quad_base.at(rk_in),
                                  chan.at(n.in_tensors[0]), plan);
            } else if (op == "Convolution") {
                const uint32_t rk_in = make_res_key(n.h_in, n.w_in, n.is_1d_tokens);
                const uint32_t rk_out = allocs.at(id).res_key;
                const uint64_t dst = place(n, id, n.cout);
                emit_conv_waves(n, cfg[i], rk_in, rk_out, dst, s2d_base, chan, plan);
            } else if (op == "SparseWave") {
                const uint32_t rk_in = make_res_key(n.h_in, n.w_in, true);
                const uint32_t rk_out = allocs.at(id).res_key;
                const uint64_t dst = place(n, id, n.cout);
                emit_sparse_wave(n, rk_in, rk_out, dst, chan, plan);
            } else if (op == "PrunedWave") {
                const uint32_t rk_in = make_res_key(n.h_in, n.w_in, true);
                const uint32_t rk_out = allocs.at(id).res_key;
                const uint64_t dst = place(n, id, n.cout);
                emit_pruned_wave(n, rk_in, rk_out, dst, chan, plan);
            }
        }
        auto it = chan.find(default_output_tensor);
        if (it != chan.end()) {
            const Shape3D s = shapes.at(default_output_tensor);
            plan.output_off = it->second[0];
            plan.logical_output_c = plan.output_c = s.c;
            plan.output_h = s.h;
            plan.output_w = s.w;
            plan.output_res_key = make_res_key(s.h, s.w, s.is_1d);
        }
    }

  public:
    std::vector<K44IRNode> nodes;
    std::string default_output_tensor = "out0";
    K44CompileOptions opts;
    K44WavePlan compiled_plan;
    bool is_compiled = false;
    std::string cached_summary_json;
    std::string last_error;

    void clear() {
        nodes.clear();
        default_output_tensor = "out0";
        is_compiled = false;
        cached_summary_json.clear();
    }

    void append_node_to_graph(K44IRNode &&n, bool update_default_output = true) {
        if (update_default_output && !n.out_tensors.empty())
            default_output_tensor = n.out_tensors[0];
        nodes.push_back(std::move(n));
        is_compiled = false;
    }

    // Interleaves row-major [Cout][B] fp16 weights into the WMMA block order (on-disk format),
    // stores indices and biases, and re-bases fp16-element indices on a 64-aligned x_base_off
    // when the largest real index reaches 0x70000000 (ref :1031-1076).
    static void pack_wave_buffers(K44ExecCmd &c, const std::vector<uint16_t> &w,
                                  const std::vector<uint32_t> &idx,
                                  const std::vector<uint16_t> &bias, K44WavePlan &plan,
                                  const std::vector<uint16_t> &cout_map = {}) {
        const size_t w_bytes = (size_t)c.Cout * c.B * 2u;
        plan.total_w_bytes += w_bytes;
        plan.total_idx_bytes += idx.size() * 4u + bias.size() * 2u + cout_map.size() * 2u;
        if (!w.empty()) {
            c.h_w_wmma.resize(w_bytes / 16u);
            convert_raw_to_wmma(c.h_w_wmma.data(), reinterpret_cast<const uint4_host *>(w.data()),
                                c.Cout, c.B / 8u);
        }
        c.h_idx = idx;
        c.x_base_off = 0u;
        if (c.idx_mode == 0u && !c.h_idx.empty() && c.B && c.B_raw) {
            const size_t rows = c.h_idx.size() / c.B;
            uint32_t lo = 0xffffffffu, hi = 0u;
            for (size_t r = 0; r < rows; ++r)
                for (uint32_t s = 0; s < c.B_raw; ++s) {
                    lo = std::min(lo, c.h_idx[r * c.B + s]);
                    hi = std::max(hi, c.h_idx[r * c.B + s]);
                }
            if (hi >= 0x70000000u && lo != 0xffffffffu) {
                const uint32_t base = lo & ~63u;
                c.x_base_off = base;
                for (size_t r = 0; r < rows; ++r)
                    for (uint32_t s = 0; s < c.B; ++s) {
                        uint32_t &v = c.h_idx[r * c.B + s];
                        v = s < c.B_raw ? v - base : 0u;
                    }
            }
        }
        c.h_bias = bias;
        c.h_cout_map = cout_map;
        c.has_cout_map = !cout_map.empty();
    }

    void add_input(const std::string &name, uint32_t ch, uint32_t h, uint32_t w,
                   bool is_1d = false) {
        K44IRNode n;
        n.op_type = "Input";
        n.name = name;
        n.out_tensors = {name};
        n.cin = n.cout = ch;
        n.h_in = n.h_out = h;
        n.w_in = n.w_out = w;
        n.is_1d_tokens = is_1d || (h == 1u && (w < 4u || w % 4u != 0u));
        append_node_to_graph(std::move(n));
    }

    void add_flatten(const std::string &name, const std::string &in, const std::string &out) {
        K44IRNode n;
        n.op_type = "Flatten";
        n.name = name;
        n.in_tensors = {in};
        n.out_tensors = {out};
        append_node_to_graph(std::move(n));
    }

    void add_rmsnorm(const std::string &name, const std::string &in, const std::string &out,
                     uint32_t dim, float eps, const float *gamma, bool pre_folded = false) {
        K44IRNode n;
        n.op_type = "RMSNorm";
        n.name = name;
        n.in_tensors = {in};
        n.out_tensors = {out};
        n.cin = n.cout = dim;
        n.eps = eps;
        n.gamma_folded = pre_folded;
        n.bias_f32.resize(dim);
        n.bias_f16.resize(dim);
        for (uint32_t i = 0; i < dim; ++i) {
            n.bias_f32[i] = gamma ? gamma[i] : 1.0f;
            n.bias_f16[i] = float_to_half(n.bias_f32[i]);
        }
        append_node_to_graph(std::move(n));
    }

  private:
    K44IRNode conv_node(const std::string &name, const std::string &in, const std::string &out,
                        uint32_t cin, uint32_t cout, uint32_t kh, uint32_t kw, uint32_t stride,
                        uint32_t pad, K44Act act, const std::string &res) {
        K44IRNode n;
        n.op_type = "Convolution";
        n.name = name;
        n.in_tensors = {in};
        n.out_tensors = {out};
        n.cin = cin;
        n.cout = cout;
        n.kh = kh;
        n.kw = kw;
        n.stride = stride;
        n.pad = pad;
        n.act = act;
        n.residual_tensor = res;
        return n;
    }

  public:
    void add_conv2d(const std::string &name, const std::string &in, const std::string &out,
                    uint32_t cin, uint32_t cout, uint32_t kh, uint32_t kw, uint32_t stride,
                    uint32_t pad, K44Act act, const float *w, const float *b,
                    const std::string &res = "") {
        K44IRNode n = conv_node(name, in, out, cin, cout, kh, kw, stride, pad, act, res);
        const size_t sz = (size_t)cout * cin * kh * kw;
        n.weights_f32.assign(sz, 0.0f);
        n.weights_f16.assign(sz, 0u);
        if (w)
            for (size_t i = 0; i < sz; ++i) {
                n.weights_f32[i] = w[i];
                n.weights_f16[i] = float_to_half(w[i]);
            }
        init_node_bias(n, cout, b);
        append_node_to_graph(std::move(n));
    }

    void add_conv2d_f16(const std::string &name, const std::string &in, const std::string &out,
                        uint32_t cin, uint32_t cout, uint32_t kh, uint32_t kw, uint32_t stride,
                        uint32_t pad, K44Act act, const uint16_t *w, const float *b,
                        const std::string &res = "") {
        K44IRNode n = conv_node(name, in, out, cin, cout, kh, kw, stride, pad, act, res);
        const size_t sz = (size_t)cout * cin * kh * kw;
        n.weights_f16.assign(sz, 0u);
        if (w) std::memcpy(n.weights_f16.data(), w, sz * 2u);
        init_node_bias(n, cout, b);
        append_node_to_graph(std::move(n));
    }

    void add_linear_bf16(const std::string &name, const std::string &in, const std::string &out,
                         uint32_t din, uint32_t dout, K44Act act, const uint16_t *w,
                         const float *b, const std::string &res = "") {
        K44IRNode n = conv_node(name, in, out, din, dout, 1u, 1u, 1u, 0u, act, res);
        n.weights_f16.assign((size_t)dout * din, 0u);
        if (w)
            for (size_t i = 0; i < n.weights_f16.size(); ++i)
                n.weights_f16[i] = float_to_half(bf16_to_float(w[i]));
        init_node_bias(n, dout, b);
        append_node_to_graph(std::move(n));
    }

    void add_upconv2x2(const std::string &name, const std::string &in, const std::string &out,
                       uint32_t cin, uint32_t cout, const float *w, const float *b) {
        K44IRNode n;
        n.op_type = "Deconvolution";
        n.name = name;
        n.in_tensors = {in};
        n.out_tensors = {out};
        n.cin = cin;
        n.cout = cout;
        n.kh = n.kw = n.stride = 2u;
        const size_t sz = (size_t)cout * cin * 4u;
        n.weights_f32.assign(sz, 0.0f);
        n.weights_f16.assign(sz, 0u);
        if (w)
            for (size_t i = 0; i < sz; ++i) {
                n.weights_f32[i] = w[i];
                n.weights_f16[i] = float_to_half(w[i]);
            }
        init_node_bias(n, cout, b);
        append_node_to_graph(std::move(n));
    }

    void add_maxpool(const std::string &name, const std::string &in, const std::string &out,
                     uint32_t k, uint32_t stride, uint32_t pad) {
        K44IRNode n;
        n.op_type = "Pooling";
        n.name = name;
        n.in_tensors = {in};
        n.out_tensors = {out};
        n.kh = n.kw = k;
        n.stride = stride;
        n.pad = pad;
        append_node_to_graph(std::move(n));
    }

    void add_upsample2x(const std::string &name, const std::string &in, const std::string &out) {
        K44IRNode n;
        n.op_type = "Interp";
        n.name = name;
        n.in_tensors = {in};
        n.out_tensors = {out};
        append_node_to_graph(std::move(n));
    }

    void add_split(const std::string &name, const std::string &in,
                   const std::vector<std::string> &outs) {
        K44IRNode n;
        n.op_type = "Split";
        n.name = name;
        n.in_tensors = {in};
        n.out_tensors = outs;
        append_node_to_graph(std::move(n), false);
    }

    void add_slice(const std::string &name, const std::string &in,
                   const std::vector<std::string> &outs, const std::vector<uint32_t> &sizes = {}) {
        K44IRNode n;
        n.op_type = "Slice";
        n.name = name;
        n.in_tensors = {in};
        n.out_tensors = outs;
        n.slice_sizes = sizes;
        append_node_to_graph(std::move(n), false);
    }

    void add_concat(const std::string &name, const std::vector<std::string> &ins,
                    const std::string &out) {
        K44IRNode n;
        n.op_type = "Concat";
        n.name = name;
        n.in_tensors = ins;
        n.out_tensors = {out};
        append_node_to_graph(std::move(n));
    }

    void add_swiglu_mul(const std::string &name, const std::string &gate, const std::string &up,
                        const std::string &out) {
        K44IRNode n;
        n.op_type = "SwiGLU";
        n.name = name;
        n.in_tensors = {gate, up};
        n.out_tensors = {out};
        append_node_to_graph(std::move(n));
    }

    void add_rope_gqa_attention(const std::string &name, const std::string &q,
                                const std::string &k, const std::string &v,
                                const std::string &out, uint32_t h_q, uint32_t h_kv,
                                uint32_t head_dim, float theta = 10000.0f, bool llama3 = false) {
        K44IRNode n;
        n.op_type = "RoPEAttention";
        n.name = name;
        n.in_tensors = {q, k, v};
        n.out_tensors = {out};
        n.h_q = h_q;
        n.h_kv = h_kv;
        n.head_dim = head_dim;
        n.rope_theta = theta;
        n.llama3_rope_scaling = llama3;
        n.cin = n.cout = h_q * head_dim;
        append_node_to_graph(std::move(n));
    }

    // Build extension: wave of `cout` neurons; neurons [r*cluster, (r+1)*cluster) share index
    // row r, which lists the input channel read by each of the fan_in synapses.
    // rows: [cout/cluster][fan_in]; w_f16: [cout][fan_in]; bias_f16: [cout] (nullable).
    void add_sparse_wave(const std::string &name, const std::string &in, const std::string &out,
                         uint32_t cout, uint32_t fan_in, uint32_t cluster, const uint32_t *rows,
                         const uint16_t *w_f16, const uint16_t *bias_f16, K44Act act,
                         const std::string &res = "", uint32_t seg_len = 0u) {
        if (cout == 0u || fan_in == 0u || cluster == 0u || cout % cluster != 0u || !rows ||
            !w_f16)
            throw std::invalid_argument("add_sparse_wave: need cout, fan_in > 0, cluster | cout, "
                                        "index rows and weights");
        K44IRNode n;
        n.op_type = "SparseWave";
        n.name = name;
        n.in_tensors = {in};
        n.out_tensors = {out};
        n.cout = cout;
        n.fan_in = fan_in;
        n.cluster = cluster;
        n.seg_len = seg_len;
        n.act = act;
        n.residual_tensor = res;
        n.rows.assign(rows, rows + (size_t)(cout / cluster) * fan_in);
        n.weights_f16.assign(w_f16, w_f16 + (size_t)cout * fan_in);
        n.bias_f16.assign(cout, 0u);
        if (bias_f16) std::memcpy(n.bias_f16.data(), bias_f16, cout * 2u);
        append_node_to_graph(std::move(n));
    }

    // Build extension: dendritic-cluster form — index row r is K segments of S consecutive input
    // channels starting at starts[r*K + k].
    void add_cluster_wave(const std::string &name, const std::string &in, const std::string &out,
                          uint32_t cout, uint32_t K, uint32_t S, uint32_t cluster,
                          const uint32_t *starts, const uint16_t *w_f16,
                          const uint16_t *bias_f16, K44Act act, const std::string &res = "") {
        if (K == 0u || S == 0u || cluster == 0u || cout % cluster != 0u || !starts)
            throw std::invalid_argument("add_cluster_wave: need K, S > 0 and cluster | cout");
        const size_t n_rows = cout / cluster, fan = (size_t)K * S;
        std::vector<uint32_t> rows(n_rows * fan);
        for (size_t r = 0; r < n_rows; ++r)
            for (uint32_t k = 0; k < K; ++k)
                for (uint32_t s = 0; s < S; ++s) rows[r * fan + (size_t)k * S + s] = starts[r * K + k] + s;
        add_sparse_wave(name, in, out, cout, (uint32_t)fan, cluster, rows.data(), w_f16, bias_f16,
                        act, res, S);
    }

    // Build extension: projection whose neurons each keep their own K dendritic clusters of S
    // consecutive input channels (starts: [cout][K], w_f16: [cout][K*S] in the same cluster
    // order).  Compiled into tiles of `tile` neurons for dense MFMA tiles:
    //   1. each neuron's clusters are sorted by start (weight segments move with them);
    //   2. pattern-sorted cutting: neurons are grouped by identical cluster pattern (groups in
    //      lexicographic order, neurons of a group in index order), every group contributes
    //      floor(n / tile) full tiles of its own pattern, and the remainders of all groups, in
    //      group order, are cut into tiles of `tile` slots (the last one partly empty); with at
    //      most kMaxPackClusters distinct clusters over all neurons, pack_union_tiles' tiles
    //      replace these unless their largest union (then their total) is larger;
    //   3. a tile's index row is the sorted union of its neurons' clusters;
    //   4. tiles are gathered into one sub-wave per union size (ascending); a neuron's weights
    //      are zero on the clusters of the union it does not keep; each sub-wave's cout_map
    //      sends slot j to the neuron's own output channel (0xFFFF: empty slot).
    // The output keeps the caller's channel order; the cout_map epilogue is y = act(v + r).
    void add_pruned_wave(const std::string &name, const std::string &in, const std::string &out,
                         uint32_t cout, uint32_t K, uint32_t S, uint32_t tile,
                         const uint32_t *starts, const uint16_t *w_f16, const uint16_t *bias_f16,
                         K44Act act, const std::string &res = "") {
        if (cout == 0u || cout >= 0xffffu || K == 0u || S == 0u || tile == 0u || !starts ||
            !w_f16)
            throw std::invalid_argument("add_pruned_wave: need 0 < cout < 65535, K, S, tile > 0, "
                                        "cluster starts and weights");
        const size_t fan = (size_t)K * S;
        // 1. per-neuron sorted pattern + the source cluster of each sorted position
        std::vector<uint32_t> pat((size_t)cout * K), src((size_t)cout * K);
        for (uint32_t j = 0; j < cout; ++j) {
            uint32_t *pj = &pat[(size_t)j * K], *sj = &src[(size_t)j * K];
            std::iota(sj, sj + K, 0u);
            std::sort(sj, sj + K, [&](uint32_t a, uint32_t b) {
                return starts[(size_t)j * K + a] < starts[(size_t)j * K + b];
            });
            for (uint32_t k = 0; k < K; ++k) {
                pj[k] = starts[(size_t)j * K + sj[k]];
                if (k && pj[k] < pj[k - 1] + S)
                    throw std::invalid_argument("add_pruned_wave '" + name +
                                                "': clusters of a neuron overlap");
            }
        }
        // 2-3. tiles; each tile = slots (neuron or -1) + union row
        struct Tile {
            std::vector<int64_t> slots;
            std::vector<uint32_t> uni;
        };
        std::vector<Tile> tiles;
        std::vector<uint32_t> univ(pat.begin(), pat.end());
        std::sort(univ.begin(), univ.end());
        univ.erase(std::unique(univ.begin(), univ.end()), univ.end());
        // pattern-sorted cutting: groups by pattern (lexicographic), full tiles per group, then
        // the groups' remainders in group order
        std::vector<std::vector<uint32_t>> chosen;
        {
            std::map<std::vector<uint32_t>, std::vector<uint32_t>> groups;
            for (uint32_t j = 0; j < cout; ++j)
                groups[std::vector<uint32_t>(pat.begin() + (size_t)j * K,
                                             pat.begin() + (size_t)(j + 1) * K)]
                    .push_back(j);
            std::vector<uint32_t> rest;
            for (const auto &g : groups) {
                const size_t full = g.second.size() / tile;
                for (size_t f = 0; f < full; ++f)
                    chosen.emplace_back(g.second.begin() + f * tile,
                                        g.second.begin() + (f + 1) * tile);
                rest.insert(rest.end(), g.second.begin() + full * tile, g.second.end());
            }
            for (size_t b = 0; b < rest.size(); b += tile)
                chosen.emplace_back(rest.begin() + b, rest.begin() + std::min(rest.size(), b + tile));
        }
        if (univ.size() <= kMaxPackClusters) {
            // bounded unions over few distinct clusters (pack_union_tiles), unless their largest
            // union (then their total) is larger than the cutting's
            std::vector<uint32_t> pm(cout, 0u);
            for (uint32_t j = 0; j < cout; ++j)
                for (uint32_t k = 0; k < K; ++k)
                    pm[j] |= 1u << (std::lower_bound(univ.begin(), univ.end(),
                                                     pat[(size_t)j * K + k]) -
                                    univ.begin());
            const uint32_t n_tiles = (cout + tile - 1u) / tile;
            auto packed = pack_union_tiles(pm, (uint32_t)univ.size(), tile, 4u * n_tiles + 64u);
            auto cost = [&](const std::vector<std::vector<uint32_t>> &ts) {
                uint32_t mx = 0, sum = 0;
                for (const auto &t : ts) {
                    uint32_t m = 0;
                    for (uint32_t j : t) m |= pm[j];
                    const uint32_t u = (uint32_t)__builtin_popcount(m);
                    mx = std::max(mx, u);
                    sum += u;
                }
                return std::make_pair(mx, sum);
            };
            if (cost(packed) <= cost(chosen)) chosen = std::move(packed);
        }
        for (const auto &js : chosen) {
            Tile t;
            std::set<uint32_t> u;
            for (uint32_t j : js) {
                t.slots.push_back(j);
                u.insert(pat.begin() + (size_t)j * K, pat.begin() + (size_t)(j + 1) * K);
            }
            t.slots.resize(tile, -1);
            t.uni.assign(u.begin(), u.end());
            tiles.push_back(std::move(t));
        }
        // 4. one sub-wave per union size
        std::map<size_t, std::vector<size_t>> by_size;
        for (size_t i = 0; i < tiles.size(); ++i) by_size[tiles[i].uni.size()].push_back(i);
        K44IRNode n;
        n.op_type = "PrunedWave";
        n.name = name;
        n.in_tensors = {in};
        n.out_tensors = {out};
        n.cout = cout;
        n.cluster = tile;
        n.seg_len = S;
        n.fan_in = (uint32_t)fan;
        n.act = act;
        n.residual_tensor = res;
        n.nnz = (uint64_t)cout * fan;
        for (const auto &bs : by_size) {
            const uint32_t U = (uint32_t)bs.first;
            n.part_tiles.push_back((uint32_t)bs.second.size());
            n.part_k.push_back(U);
            for (size_t ti : bs.second) {
                const Tile &t = tiles[ti];
                n.rows.insert(n.rows.end(), t.uni.begin(), t.uni.end());
                for (int64_t j : t.slots) {
                    const size_t at = n.weights_f16.size();
                    n.weights_f16.resize(at + (size_t)U * S, 0u);
                    if (j < 0) {
                        n.bias_f16.push_back(0u);
                        n.cout_map.push_back(0xffffu);
                        continue;
                    }
                    const uint32_t *pj = &pat[(size_t)j * K], *sj = &src[(size_t)j * K];
                    for (uint32_t k = 0, q = 0; k < U; ++k) {
                        while (q < K && pj[q] < t.uni[k]) ++q;
                        if (q < K && pj[q] == t.uni[k])
                            std::memcpy(&n.weights_f16[at + (size_t)k * S],
                                        &w_f16[(size_t)j * fan + (size_t)sj[q] * S], S * 2u);
                    }
                    n.bias_f16.push_back(bias_f16 ? bias_f16[j] : (uint16_t)0u);
                    n.cout_map.push_back((uint16_t)j);
                }
            }
        }
        append_node_to_graph(std::move(n));
    }

    // Build extension: causal depth-wise token mix y[c][t] = sum_{i<rf} mu[c][i] x[c][t-i] within
    // requests of seq_len tokens (prefill), or one token per request with carried state (decode).
    void add_token_shift(const std::string &name, const std::string &in, const std::string &out,
                         uint32_t dim, uint32_t rf, uint32_t seq_len, const uint16_t *mu_f16,
                         bool decode) {
        if (rf == 0u || rf > 9u || seq_len == 0u || !mu_f16 || dim == 0u)
            throw std::invalid_argument("add_token_shift: need 1 <= rf <= 9, seq_len > 0, mix");
        K44IRNode n;
        n.op_type = "TokenShift";
        n.name = name;
        n.in_tensors = {in};
        n.out_tensors = {out};
        n.rf = rf;
        n.seq_len = seq_len;
        n.decode_state = decode;
        n.table.assign(mu_f16, mu_f16 + (size_t)dim * rf);
        append_node_to_graph(std::move(n));
    }

    // Build extension: y[c][t] = table[id[t]][c]; ids come from the executor's id buffer
    // (wavec_gpu_set_ids, or the previous run's ArgMax).  `tok_in` supplies the token axis.
    void add_embedding(const std::string &name, const std::string &tok_in, const std::string &out,
                       uint32_t vocab, uint32_t dim, const uint16_t *table_f16) {
        if (vocab == 0u || dim == 0u || !table_f16)
            throw std::invalid_argument("add_embedding: need vocab, dim and a table");
        K44IRNode n;
        n.op_type = "Embedding";
        n.name = name;
        n.in_tensors = {tok_in};
        n.out_tensors = {out};
        n.vocab = vocab;
        n.cout = dim;
        n.table.assign(table_f16, table_f16 + (size_t)vocab * dim);
        append_node_to_graph(std::move(n));
    }

    // Build extension: id[t] = argmax_c x[c][t] into the executor's id buffer.
    void add_argmax(const std::string &name, const std::string &in, const std::string &out) {
        K44IRNode n;
        n.op_type = "ArgMax";
        n.name = name;
        n.in_tensors = {in};
        n.out_tensors = {out};
        append_node_to_graph(std::move(n), false);
    }

    const K44WavePlan &compile() {
        K44WavePlan plan;
        std::map<std::string, Shape3D> shapes;
        std::vector<K44WaveConfig> cfg;
        std::map<int, PhysAlloc> allocs;
        std::vector<int> out_aid;
        std::map<uint32_t, uint64_t> s2d_base, quad_base;
        std::map<size_t, std::pair<uint64_t, uint64_t>> kv_offs;
        uint64_t probs_off = 0u;
        pass1_infer_shapes(plan, shapes);
        pass2_fold_rmsnorm(plan);
        pass3_build_layouts(plan, shapes, cfg);
        pass4_allocate_canvas(plan, cfg, allocs, out_aid, s2d_base, quad_base, kv_offs,
                              probs_off);
        pass5_emit_commands(plan, shapes, cfg, allocs, out_aid, s2d_base, quad_base, kv_offs,
                            probs_off);
        compiled_plan = std::move(plan);
        is_compiled = true;
        build_summary_json();
        return compiled_plan;
    }

    // Summary JSON: the reference's keys and formats (ref :1345-1405); sparse waves add
    // "seg_len" and "idx_mode" to their command line.
    void build_summary_json() {
        const K44WavePlan &p = compiled_plan;
        char hdr[2048];
        std::snprintf(
            hdr, sizeof(hdr),
            "{\n  \"batch_size\": %u,\n  \"num_waves\": %d,\n  \"num_cmds\": %zu,\n"
            "  \"canvas_elems\": %zu,\n  \"canvas_bytes\": %llu,\n  \"kv_cache_elems\": %zu,\n"
            "  \"total_w_bytes\": %zu,\n  \"total_idx_bytes\": %zu,\n"
            "  \"single_frame_gflops\": %.6g,\n  \"total_gflops\": %.6g,\n"
            "  \"single_frame_gsyn\": %.6g,\n  \"total_gsyn\": %.6g,\n"
            "  \"num_folded_rmsnorms\": %d,\n  \"num_eliminated_concats\": %d,\n"
            "  \"num_eliminated_splits\": %d,\n  \"num_zero_copy_flattens\": %d,\n"
            "  \"input_shape\": [%u, %u, %u],\n  \"output_shape\": [%u, %u, %u],\n"
            "  \"max_B_per_wave\": %u,\n  \"target_profile\": \"%s\",\n"
            "  \"target_num_cus\": %u,\n  \"persistent_neurons\": %s,\n"
            "  \"reuse_canvas\": %s,\n  \"cmds\": [\n",
            p.batch_size, p.num_wave_dispatches, p.cmds.size(), p.canvas_elems,
            (unsigned long long)(p.canvas_elems * 2ULL), p.kv_cache_elems, p.total_w_bytes,
            p.total_idx_bytes, p.single_frame_gflops, p.total_gflops,
            p.single_frame_gflops * 0.5, p.total_gflops * 0.5, p.num_folded_rmsnorms,
            p.num_eliminated_concats, p.num_eliminated_splits, p.num_zero_copy_flattens,
            p.input_c, p.input_h, p.input_w, p.logical_output_c, p.output_h, p.output_w,
            opts.max_B_per_wave, opts.hw_profile.name.c_str(), opts.hw_profile.num_cus,
            opts.reuse_canvas ? "false" : "true", opts.reuse_canvas ? "true" : "false");
        std::string js(hdr);
        js.reserve(js.size() + p.cmds.size() * 300u + 16u);
        for (size_t i = 0; i < p.cmds.size(); ++i) {
            const K44ExecCmd &c = p.cmds[i];
            // Build-extension keys (the reference's readers ignore unknown keys).
            char extra[256] = "";
            size_t ne = 0;
            auto add = [&](const char *fmt, unsigned long long a, unsigned long long b = 0,
                           unsigned long long c3 = 0, unsigned long long d = 0) {
                if (ne < sizeof(extra))
                    ne += (size_t)std::snprintf(extra + ne, sizeof(extra) - ne, fmt, a, b, c3, d);
            };
            if (c.seg_len || c.idx_mode)
                add(", \"seg_len\": %llu, \"idx_mode\": %llu", c.seg_len, c.idx_mode);
            if (c.has_residual) add(", \"res_off\": %llu", (unsigned long long)c.res_off);
            if (c.type == K44CmdType::SWIGLU_MUL_1D)
                add(", \"src2_off\": %llu", (unsigned long long)c.src2_off);
            if (c.type == K44CmdType::TOKEN_SHIFT_1D)
                add(", \"rf\": %llu, \"seq_len\": %llu, \"decode\": %llu, \"state_off\": %llu",
                    c.rf, c.seq_len, c.decode_state ? 1u : 0u, (unsigned long long)c.state_off);
            char line[1024];
            std::snprintf(
                line, sizeof(line),
                "    {\"idx\": %zu, \"name\": \"%s\", \"type\": \"%s\", \"Cin\": %u, \"Cout\": %u, "
                "\"logical_Cout\": %u, \"B\": %u, \"B_raw\": %u, \"S\": %u, \"act\": \"%s\", "
                "\"has_residual\": %s, \"has_self_read\": %s, \"subwave\": [%u, %u], \"h_out\": "
                "%u, \"w_out\": %u, \"src_off\": %llu, \"y_off\": %llu, \"gflops\": %.6g%s}%s\n",
                i, c.name.c_str(), cmd_type_str(c.type), c.Cin, c.Cout, c.logical_Cout, c.B,
                c.B_raw, c.cluster_size, act_str(c.act), c.has_residual ? "true" : "false",
                c.has_self_read ? "true" : "false", c.subwave_idx, c.num_subwaves, c.h_out,
                c.w_out, (unsigned long long)c.src_off, (unsigned long long)c.y_off, c.gflops,
                extra, i + 1 < p.cmds.size() ? "," : "");
            js += line;
        }
        js += "  ]\n}\n";
        cached_summary_json = std::move(js);
    }
};

}  // namespace k44_host
