// k44_plan_types.hpp — host plan types of the SNNtome wave boundary (namespace k44_host).
//
// Same public API as the reference's wavec/k44_plan_types.hpp (names, enum values, struct
// fields, layout formulas), implemented independently for an MI355X executor.  Differences,
// all additive:
//   * K44Act::GELU = 5 (erf form).
//   * K44ExecCmd / K44WavePlan canvas offsets are 64-bit, so one canvas may exceed 2^32 fp16
//     elements (a 40M-position x 256-token substrate is 10.2 G elements).
//   * K44ExecCmd::idx_mode: 0 = h_idx holds fp16-element canvas offsets (reference meaning);
//     1 = h_idx holds substrate row indices, canvas offset = x_base_off + idx * idx_stride.
//   * K44ExecCmd::seg_len: segment length hint (positions per dendritic cluster) of sparse waves.
//   * Hardware preset "mi355x" (also what "auto" resolves to in this build).
#pragma once
#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <set>
#include <string>
#include <vector>

namespace k44_host {

// ------------------------------------------------------------------------------------------------
// 1. fp16 / bf16 host conversion (k44_plan_types.hpp:21-94 of the reference): IEEE binary16,
//    round-half-even; NaN keeps the top payload bits and forces the low bit on.
// ------------------------------------------------------------------------------------------------
static inline uint16_t float_to_half(float f) {
    uint32_t u;
    std::memcpy(&u, &f, sizeof(u));
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t mag = u & 0x7fffffffu;
    if (mag >= 0x7f800000u) {  // Inf / NaN
        return (uint16_t)(mag == 0x7f800000u ? (sign | 0x7c00u)
                                             : (sign | 0x7c00u | ((mag & 0x7fffffu) >> 13) | 1u));
    }
    if (mag < 0x38800000u) {   // below the smallest normal half (2^-14)
        if (mag < 0x33000000u) return (uint16_t)sign;  // < 2^-25: rounds to +-0
        const uint32_t shift = 126u - (mag >> 23);
        const uint32_t full = (mag & 0x7fffffu) | 0x800000u;
        uint32_t q = full >> shift;
        const uint32_t rem = full & ((1u << shift) - 1u), tie = 1u << (shift - 1u);
        q += (rem > tie || (rem == tie && (q & 1u))) ? 1u : 0u;
        return (uint16_t)(sign | q);
    }
    const uint32_t rebased = mag - 0x38000000u;  // exponent bias 127 -> 15
    uint32_t q = rebased >> 13;
    const uint32_t rem = rebased & 0x1fffu;
    q += (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ? 1u : 0u;
    return (uint16_t)(sign | std::min(q, 0x7c00u));
}

static inline float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t u;
    if (e == 0x1fu) {
        u = sign | 0x7f800000u | (m << 13);
    } else if (e) {
        u = sign | ((e + 112u) << 23) | (m << 13);
    } else if (!m) {
        u = sign;
    } else {
        const float v = (float)m * (1.0f / 16777216.0f);
        std::memcpy(&u, &v, sizeof(u));
        u |= sign;
    }
    float f;
    std::memcpy(&f, &u, sizeof(f));
    return f;
}

static inline float bf16_to_float(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, sizeof(f));
    return f;
}

struct alignas(16) uint4_host {
    uint32_t x, y, z, w;
};

enum class K44Act : int { NONE = 0, RELU = 1, SIGMOID = 2, SILU = 3, LEAKY_RELU = 4, GELU = 5 };

enum class K44CmdType : int {
    K44_WAVE = 0,
    S2D_2X2 = 1,
    MAXPOOL_2X2 = 2,
    MAXPOOL_5X5 = 3,
    UPSAMPLE_2X = 4,
    SCATTER_UP2X2 = 5,
    RMSNORM_1D = 7,
    SWIGLU_MUL_1D = 8,
    ROPE_GQA_ATTN_1D = 9,
    // build extensions (1-D token ops of LLM-shaped wave plans)
    TOKEN_SHIFT_1D = 10,
    EMBED_1D = 11,
    ARGMAX_1D = 12
};

static inline const char *cmd_type_str(K44CmdType t) {
    static const char *const names[] = {"K44_WAVE",       "S2D_2X2",        "MAXPOOL_2X2",
                                        "MAXPOOL_5X5",    "UPSAMPLE_2X",    "SCATTER_UP2X2",
                                        "UNKNOWN",        "RMSNORM_1D",     "SWIGLU_MUL_1D",
                                        "ROPE_GQA_ATTN_1D", "TOKEN_SHIFT_1D", "EMBED_1D",
                                        "ARGMAX_1D"};
    const int i = (int)t;
    return (i >= 0 && i <= 12) ? names[i] : "UNKNOWN";
}

static inline const char *act_str(K44Act a) {
    static const char *const names[] = {"NONE", "RELU", "SIGMOID", "SILU", "LEAKY_RELU", "GELU"};
    const int i = (int)a;
    return (i >= 0 && i <= 5) ? names[i] : "NONE";
}

// Cout padding: multiple of 16, at least 16.  Fan-in padding: multiple of 32, at least 64.
static inline uint32_t round_up_16(uint32_t v) { return std::max(16u, (v + 15u) & ~15u); }
static inline uint32_t round_up_32(uint32_t v) { return std::max(64u, (v + 31u) & ~31u); }

// Cluster (index-row sharing) size for a dense wave (k44_plan_types.hpp:167-186): a forced size
// is halved until it divides cout (not below 16); otherwise 128 when cout % 128 == 0 and
// (cout >= 640 or few tiles), else the largest of 64/32/16 dividing cout.
static inline uint32_t choose_cluster_size(uint32_t cout, uint32_t num_tiles,
                                           uint32_t force_cluster_size = 0u) {
    for (uint32_t s = force_cluster_size; s >= 16u; s >>= 1u)
        if (cout % s == 0u) return s;
    if (cout % 128u == 0u && (cout >= 640u || num_tiles <= 64u)) return 128u;
    for (uint32_t s : {64u, 32u})
        if (cout % s == 0u) return s;
    return 16u;
}

// ------------------------------------------------------------------------------------------------
// 2. Hardware profiles.  As in the reference, they are reported in the compile summary but do
//    not change the wave configuration (k44_plan_types.hpp:328-343).
// ------------------------------------------------------------------------------------------------
struct K44HardwareProfile {
    std::string name = "mi355x";
    uint32_t num_cus = 256u;
    uint32_t max_clusters_cta = 4u;
    double r_tc_syn_s = 1.25e15;
    double bw_vram_bytes_s = 8.0e12;
    double bw_cache_bytes_s = 17.0e12;
    double bw_l1_bytes_s = 60.0e12;
    double v_cache_win = 256.0 * 1024.0 * 1024.0;
    double v_cache_budget = 192.0 * 1024.0 * 1024.0;
    double cache_gamma = 2.0;
    double k_pipe_half = 32.0;
    double w_cta_half = 0.80;
    double occ_waves_half = 4.0;
    double chunk_launch_s = 3.5e-6;
    double gather_subtile_pen = 0.04;
    uint32_t max_b_per_wave = 0u;

    static K44HardwareProfile make(const char *n, uint32_t cus, uint32_t clusters, double syn,
                                   double vram, double cache, double l1, double win,
                                   double budget) {
        K44HardwareProfile p;
        p.name = n;
        p.num_cus = cus;
        p.max_clusters_cta = clusters;
        p.r_tc_syn_s = syn;
        p.bw_vram_bytes_s = vram;
        p.bw_cache_bytes_s = cache;
        p.bw_l1_bytes_s = l1;
        p.v_cache_win = win;
        p.v_cache_budget = budget;
        return p;
    }

    // Preset names follow the reference (k44_plan_types.hpp:210-305) plus "mi355x".
    static K44HardwareProfile from_preset(const char *preset_str) {
        std::string p = preset_str ? preset_str : "auto";
        for (char &c : p) c = (char)std::tolower((unsigned char)c);
        const double MiB = 1024.0 * 1024.0;
        if (p.empty() || p == "auto" || p == "mi355x" || p == "gfx950" || p == "cdna4")
            return make("mi355x", 256u, 4u, 1.25e15, 8.0e12, 17.0e12, 60.0e12, 256 * MiB,
                        192 * MiB);
        if (p == "rtx6000ada" || p == "rtx6000_ada" || p == "rtx6000" || p == "ada" ||
            p == "sm_89" || p == "l40s")
            return make("rtx6000ada", 142u, 3u, 115.0e12, 795.6e9, 4078.7e9, 14000.0e9, 64 * MiB,
                        48 * MiB);
        if (p == "rtx4090" || p == "4090")
            return make("rtx4090", 128u, 3u, 125.0e12, 1008.0e9, 4200.0e9, 12800.0e9, 54 * MiB,
                        36 * MiB);
        if (p == "h100" || p == "sm_90" || p == "hopper")
            return make("h100", 132u, 3u, 350.0e12, 3350.0e9, 5500.0e9, 18000.0e9, 38 * MiB,
                        28 * MiB);
        if (p == "b200" || p == "blackwell" || p == "sm_100" || p == "sm_100a")
            return make("b200", 148u, 3u, 900.0e12, 8000.0e9, 14000.0e9, 32000.0e9, 96 * MiB,
                        64 * MiB);
        return make("rx9060xt", 32u, 2u, 27.72e12, 320.0e9, 1400.0e9, 4500.0e9, 24 * MiB,
                    16 * MiB);
    }
    static K44HardwareProfile from_preset_base(const char *preset_str) {
        return from_preset(preset_str);
    }
};

struct K44WaveConfig {
    uint32_t S1 = 64u;
    uint32_t Cout_pad1 = 64u;
    uint32_t S2 = 0u;
    uint32_t Cout_pad2 = 0u;
    uint32_t num_sub_b = 1u;
    uint32_t total_cout_pad() const { return Cout_pad1 + Cout_pad2; }
    bool is_split() const { return S2 > 0u && Cout_pad2 > 0u; }
};

static inline K44WaveConfig select_optimal_wave_config(
    uint32_t /*cin*/, uint32_t cout, uint32_t /*kh*/, uint32_t /*kw*/, uint32_t /*spatial_in*/,
    uint32_t spatial_out, uint32_t force_cluster_size = 0u,
    const K44HardwareProfile & /*hw_prof*/ = K44HardwareProfile(), uint32_t /*force_max_b*/ = 0u) {
    const uint32_t cout_pad = round_up_16(cout);
    const uint32_t s = choose_cluster_size(cout_pad, std::max(1u, spatial_out), force_cluster_size);
    return {s, cout_pad, 0u, 0u, 1u};
}

// ------------------------------------------------------------------------------------------------
// 3. RDNA4 WMMA weight order — the on-disk order of .tcff weight blocks
//    (k44_plan_types.hpp:349-394).  Vector g = (rb * B_vec16 + kb) * 32 + l (8 fp16 each) holds
//    row 16*rb + (l & 15), fp16 columns 16*kb + 8*(l >> 4) .. +8 of the row-major [Cout][B]
//    matrix.  The MI355X executor converts back to its own layouts at upload.
// ------------------------------------------------------------------------------------------------
static inline size_t wmma_src_vec(size_t g, uint32_t B_vec8) {
    const size_t B_vec16 = B_vec8 / 2u, tile = g >> 5, l = g & 31u;
    return ((tile / B_vec16) * 16u + (l & 15u)) * B_vec8 + 2u * (tile % B_vec16) + (l >> 4);
}

static inline void convert_raw_to_wmma(uint4_host *dst_wmma, const uint4_host *src_compact,
                                       uint32_t num_output_neurons, uint32_t B_vec8) {
    const size_t n = (size_t)(num_output_neurons / 16u) * (B_vec8 / 2u) * 32u;
    for (size_t g = 0; g < n; ++g) dst_wmma[g] = src_compact[wmma_src_vec(g, B_vec8)];
}

static inline void convert_wmma_to_raw(uint4_host *dst_compact, const uint4_host *src_wmma,
                                       uint32_t num_output_neurons, uint32_t B_vec8) {
    const size_t n = (size_t)(num_output_neurons / 16u) * (B_vec8 / 2u) * 32u;
    for (size_t g = 0; g < n; ++g) dst_compact[wmma_src_vec(g, B_vec8)] = src_wmma[g];
}

// ------------------------------------------------------------------------------------------------
// 4. Resolution descriptor: 64-element tile tables of a tensor layout on the canvas
//    (k44_plan_types.hpp:447-601).  Three layouts:
//    1-D tokens: channel row of ceil(W/64)*64 tokens per frame; tile t at frame_off + 64 t.
//    2-D, W % 64 == 0: W_pad = W + 8, H_pad = H + 2; X tiles pre-shifted to (ty-1, 64 tx - 1).
//    2-D otherwise: W_pad = W + 4; Y entries pack (offset >> 2) | lane-mask << 16.
// ------------------------------------------------------------------------------------------------
struct K44ResDesc {
    uint32_t H = 0, W = 0, H_pad = 0, W_pad = 0;
    uint32_t batch_size = 1;
    uint32_t tiles_per_row = 0, tiles_per_frame = 0, num_tiles = 0;
    uint32_t single_stride = 0, channel_stride = 0;
    bool needs_mask = false;
    bool is_1d_tokens = false;
    bool is_image_token64 = false;
    std::vector<uint32_t> h_tile_off_X, h_tile_off_Y, h_tile_off_X_s2;

    void init(uint32_t height, uint32_t width, bool is_1d = false, uint32_t b_frames = 1u) {
        H = height;
        W = width;
        is_1d_tokens = is_1d;
        batch_size = std::max(1u, b_frames);
        is_image_token64 = !is_1d && batch_size >= 64u && batch_size % 64u == 0u;
        h_tile_off_X_s2.clear();
        if (is_1d) {
            needs_mask = false;
            H_pad = 1u;
            tiles_per_frame = tiles_per_row = (W + 63u) / 64u;
            single_stride = W_pad = tiles_per_frame * 64u;
        } else if (W % 64u == 0u) {
            needs_mask = false;
            tiles_per_row = W / 64u;
            W_pad = W + 8u;
            H_pad = H + 2u;
            single_stride = H_pad * W_pad;
            tiles_per_frame = H * tiles_per_row;
        } else {
            needs_mask = true;
            W_pad = W + 4u;
            H_pad = H + 2u;
            tiles_per_frame = (H * W_pad + 63u) / 64u;
            tiles_per_row = 0u;
            single_stride = (2u * W_pad + tiles_per_frame * 64u + 63u) & ~63u;
        }
        num_tiles = batch_size * tiles_per_frame;
        channel_stride = batch_size * single_stride;
        h_tile_off_X.assign(num_tiles, 0u);
        h_tile_off_Y.assign(num_tiles, 0u);
        for (uint32_t f = 0; f < batch_size; ++f) {
            const uint32_t fo = f * single_stride;
            for (uint32_t t = 0; t < tiles_per_frame; ++t) {
                const uint32_t i = f * tiles_per_frame + t;
                if (is_1d) {
                    h_tile_off_X[i] = h_tile_off_Y[i] = fo + 64u * t;
                } else if (!needs_mask) {
                    const uint32_t ty = t / tiles_per_row, tx = t % tiles_per_row;
                    h_tile_off_X[i] = fo + ty * W_pad + 64u * tx + 3u;
                    h_tile_off_Y[i] = fo + (ty + 1u) * W_pad + 64u * tx + 4u;
                } else {
                    const uint32_t y1 = W_pad + 4u + 64u * t;
                    h_tile_off_X[i] = fo + y1 - W_pad - 1u;
                    uint32_t mask = 0u;
                    for (uint32_t q = 0; q < 16u; ++q) {
                        const uint32_t rel = 64u * t + 4u * q;
                        if (rel / W_pad < H && rel % W_pad < W) mask |= 1u << q;
                    }
                    h_tile_off_Y[i] = (((fo + y1) >> 2) & 0xffffu) | (mask << 16);
                }
            }
        }
    }

    // fp16 element offset of (channel, y, x, frame) inside a tensor region.
    uint32_t canvas_offset(uint32_t ch, uint32_t y, uint32_t x, uint32_t bf = 0u) const {
        if (is_1d_tokens) return ch * channel_stride + bf * single_stride + x;
        // 64-frame blocks are 64 * single_stride apart (the reference's (bf / 64) *
        // single_stride would put block 1 inside block 0's plane; equal for one block).
        if (is_image_token64)
            return ch * channel_stride + (bf / 64u) * 64u * single_stride +
                   ((y + 1u) * W_pad + x + 1u) * 64u + (bf & 63u);
        return ch * channel_stride + bf * single_stride + (y + 1u) * W_pad + 4u + x;
    }

    // Gather index of a receptive-field tap (dy, dx) for a channel based at ch_base_half.
    uint32_t tap_offset(uint32_t ch_base_half, int dy, int dx) const {
        if (is_1d_tokens) return ch_base_half + (uint32_t)dx;
        const uint32_t rel = (uint32_t)(1 + dy) * W_pad + (uint32_t)(1 + dx);
        return ch_base_half + (is_image_token64 ? rel * 64u : rel);
    }
};

struct K44ExecCmd {
    K44CmdType type = K44CmdType::K44_WAVE;
    std::string name;
    uint32_t Cout = 0;
    uint32_t logical_Cout = 0;
    uint32_t Cin = 0;
    uint32_t cluster_size = 64;
    uint32_t B = 0;
    uint32_t B_raw = 0;
    uint32_t B_vec16 = 0;
    bool has_bias = true;
    K44Act act = K44Act::NONE;
    bool has_residual = false;
    bool has_cout_map = false;
    bool has_self_read = false;
    bool needs_halo_clear = false;
    uint32_t subwave_idx = 0;
    uint32_t num_subwaves = 1;
    uint32_t weight_bits = 16;
    uint64_t y_off = 0;
    uint64_t src_off = 0;
    uint64_t src2_off = 0;
    uint64_t src3_off = 0;
    uint64_t res_off = 0;
    uint64_t x_base_off = 0;
    uint32_t res_key_in = 0;
    uint32_t res_key_out = 0;
    uint32_t h_in = 0;
    uint32_t w_in = 0;
    uint32_t h_out = 0;
    uint32_t w_out = 0;
    uint32_t h_q = 0;
    uint32_t h_kv = 0;
    uint32_t head_dim = 64;
    uint64_t kv_k_off = 0;
    uint64_t kv_v_off = 0;
    uint32_t kv_max_seq = 0;
    uint64_t attn_probs_off = 0;
    float eps = 1e-5f;
    float rope_theta = 10000.0f;
    bool llama3_rope_scaling = false;
    bool gamma_folded = false;
    double gflops = 0.0;
    // --- build extensions ---
    uint32_t idx_mode = 0;    // 0: h_idx = fp16-element offsets; 1: substrate row indices
    uint64_t idx_stride = 1;  // fp16 elements per row index (idx_mode 1)
    uint32_t seg_len = 0;     // positions per dendritic cluster (0 = unknown)
    uint32_t rf = 0;          // TOKEN_SHIFT_1D: receptive field (taps)
    uint32_t seq_len = 0;     // TOKEN_SHIFT_1D: tokens per request (prefill)
    bool decode_state = false;  // TOKEN_SHIFT_1D: one token per request, state carried
    uint64_t state_off = 0;   // TOKEN_SHIFT_1D: canvas offset of the [C][rf-1][64] state block
    std::vector<uint16_t> h_table;  // EMBED_1D: [vocab][dim] fp16; TOKEN_SHIFT_1D: [C][rf] mix
    std::vector<uint4_host> h_w_wmma;
    std::vector<uint32_t> h_idx;
    std::vector<uint16_t> h_bias;
    std::vector<uint16_t> h_cout_map;
};

struct K44CompileOptions {
    uint32_t max_B_per_wave = 0;
    bool fold_rmsnorm_gamma = true;
    bool keep_host_plan_buffers = true;
    bool reuse_canvas = false;
    uint32_t force_cluster_size = 0;
    uint32_t kv_cache_max_seq = 0;
    uint32_t batch_size = 1;
    K44HardwareProfile hw_profile = K44HardwareProfile::from_preset("auto");
};

struct K44WavePlan {
    uint32_t batch_size = 1;
    uint32_t wave_batch_size = 1;
    bool is_image_token64 = false;
    size_t canvas_elems = 0;
    size_t kv_cache_elems = 0;
    size_t total_w_bytes = 0;
    size_t total_idx_bytes = 0;
    double single_frame_gflops = 0;
    double total_gflops = 0.0;
    int num_wave_dispatches = 0;
    int num_folded_rmsnorms = 0;
    int num_eliminated_concats = 0;
    int num_eliminated_splits = 0;
    int num_zero_copy_flattens = 0;
    uint64_t input_off = 0;
    uint32_t input_c = 0;
    uint32_t input_h = 0;
    uint32_t input_w = 0;
    uint32_t input_res_key = 0;
    uint64_t output_off = 0;
    uint32_t output_c = 0;
    uint32_t logical_output_c = 0;
    uint32_t output_h = 0;
    uint32_t output_w = 0;
    uint32_t output_res_key = 0;
    bool reuse_canvas = false;
    K44HardwareProfile hw_profile = K44HardwareProfile::from_preset("auto");
    std::map<uint32_t, K44ResDesc> res_map;
    std::vector<K44ExecCmd> cmds;
};

struct K44IRNode {
    std::string op_type;
    std::string name;
    std::vector<std::string> in_tensors;
    std::vector<std::string> out_tensors;
    std::vector<uint32_t> slice_sizes;
    uint32_t cin = 0;
    uint32_t cout = 0;
    uint32_t kh = 1;
    uint32_t kw = 1;
    uint32_t stride = 1;
    uint32_t pad = 0;
    uint32_t h_in = 0;
    uint32_t w_in = 0;
    uint32_t h_out = 0;
    uint32_t w_out = 0;
    uint32_t h_q = 0;
    uint32_t h_kv = 0;
    uint32_t head_dim = 64;
    float eps = 1e-5f;
    float rope_theta = 10000.0f;
    bool llama3_rope_scaling = false;
    bool is_1d_tokens = false;
    bool gamma_folded = false;
    K44Act act = K44Act::NONE;
    std::string residual_tensor;
    std::vector<float> weights_f32;
    std::vector<uint16_t> weights_f16;
    std::vector<float> bias_f32;
    std::vector<uint16_t> bias_f16;
    // --- build extension: explicit sparse wave ("SparseWave") ---
    uint32_t fan_in = 0;         // synapses per neuron (B_raw)
    uint32_t cluster = 1;        // neurons sharing one index row
    uint32_t seg_len = 0;        // positions per dendritic cluster (hint, 0 = unknown)
    std::vector<uint32_t> rows;  // [cout/cluster][fan_in] input channel index of every synapse
    // --- build extension: pattern-sorted pruned projection ("PrunedWave"): sub-wave p has
    // part_tiles[p] tiles of `cluster` slots whose index rows are part_k[p] segments of seg_len
    // channels; rows holds the segment starts of every tile, weights_f16 / bias_f16 / cout_map the
    // slots of every sub-wave in order (cout_map 0xFFFF = empty slot, no output). ---
    std::vector<uint32_t> part_tiles, part_k;
    std::vector<uint16_t> cout_map;
    uint64_t nnz = 0;  // real synapses (cout x K x seg_len): the effective FLOP count
    // --- build extension: 1-D token ops ("TokenShift", "Embedding", "ArgMax") ---
    uint32_t rf = 0, seq_len = 0, vocab = 0;
    bool decode_state = false;
    std::vector<uint16_t> table;  // Embedding [vocab][dim]; TokenShift [C][rf]
};

}  // namespace k44_host
