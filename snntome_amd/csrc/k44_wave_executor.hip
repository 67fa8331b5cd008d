// k44_wave_executor.hip — the wavec C ABI over the executor of compiled wave plans.
//
// Replaces the reference's extern "C" frontend (wavec/k44_wave_executor.cu:642-988): the 30
// reference entry points keep their signatures, argument meaning and 0 / -1 return convention,
// and the build extensions declared in include/k44wavec.h are added.  Errors never terminate
// the process: each entry point returns -1 and records a message readable through
// wavec_last_error().  Also here: the process-wide tuning switches and the workspace of the
// allocation-free entry points.  The executor itself is k44_executor.hpp.
#include "k44_executor.hpp"

#include <map>

namespace k44_host {

namespace {
// Switch values (-1 = automatic) and their wavec_set_tuning keys, in Tune order.
std::atomic<int> g_tune[(int)Tune::Count];
const char *const kTuneKeys[(int)Tune::Count] = {
    "path", "dma", "dma_stages", "nt", "splitk", "lane8", "ksplit", "stream_kernel", "narrow",
    "narrow_chunk", "group", "group_split", "fuse", "sort", "wlds", "t64_ring", "xcd_order",
    "narrow_wgs", "narrow_reduce", "dma_prod", "program", "prog_spin_ms", "prog_trace",
    "narrow_pre", "narrow_local", "embed_refresh", "narrow_byy"};
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
    {V01, 0},          // narrow_pre
    {V01, 0},          // narrow_local
    {V01, 0},          // embed_refresh
    {V01, 0},          // narrow_byy
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

}  // namespace

namespace k44_host {

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
        ex->check_placement();
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
        ex->check_placement();
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
