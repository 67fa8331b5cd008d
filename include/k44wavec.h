/*
 * k44wavec.h — C ABI of libk44wavec.so, the MI355X (gfx950) wave executor.
 *
 * The first 30 entry points are the reference's C ABI (wavec/k44_wave_executor.cu:642-988 of
 * 7BitLogic/SNNtome) with identical names, signatures, argument meaning and return convention
 * (0 = success, -1 = failure; pointers NULL on failure).  They are what the reference's ctypes
 * binding (wavec/wavec.py:28-132) binds.  Differences in behaviour, all on error paths:
 *   - a HIP runtime error returns -1 (the reference calls exit(EXIT_FAILURE));
 *   - a plan the executor cannot run (RoPE/GQA attention, the one command kind outside this
 *     build) fails wavec_gpu_init_plan with -1 instead of silently skipping commands; 1-D token
 *     plans and 2-D spatial plans (padded-plane and 64-frame interleaved layouts, with their
 *     pools, upsampling, stride-2 and transposed convolutions) run;
 *   - the message of the last failure on the calling thread is available from wavec_last_error().
 *
 * The entry points after "build extensions" have no counterpart in the reference.
 * Plain C types only; no torch or HIP types cross this boundary.
 */
#ifndef K44WAVEC_H
#define K44WAVEC_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Activation ids (wavec/wavec.py:13-16 ACT_MAP, k44_plan_types.hpp:103); 5 = GELU (extension). */
enum { K44_ACT_NONE = 0, K44_ACT_RELU = 1, K44_ACT_SIGMOID = 2, K44_ACT_SILU = 3,
       K44_ACT_LEAKY_RELU = 4, K44_ACT_GELU = 5 };

/* ---- graph handle (k44_wave_executor.cu:644-683) ------------------------------------------- */
void *wavec_create(int max_B_per_wave, int default_S, int kv_cache_max_seq, int fold_rmsnorm_gamma);
void wavec_destroy(void *handle);
int wavec_gpu_release(void *handle);

/* ---- graph builders (k44_wave_executor.cu:685-873) ------------------------------------------ */
int wavec_add_input(void *handle, const char *name, int c, int h, int w, int is_1d);
int wavec_add_flatten(void *handle, const char *name, const char *in_tensor, const char *out_tensor);
/* w_f32: [cout][cin][kh][kw]; bias_f32 and residual_tensor may be NULL. (:704-716) */
int wavec_add_conv2d(void *handle, const char *name, const char *in_tensor, const char *out_tensor,
                     int cin, int cout, int kh, int kw, int stride, int pad, int act,
                     const float *w_f32, const float *bias_f32, const char *residual_tensor);
int wavec_add_conv2d_f16(void *handle, const char *name, const char *in_tensor,
                         const char *out_tensor, int cin, int cout, int kh, int kw, int stride,
                         int pad, int act, const uint16_t *w_f16, const float *bias_f32,
                         const char *residual_tensor);                                  /* :718-731 */
int wavec_add_linear_f32(void *handle, const char *name, const char *in_tensor,
                         const char *out_tensor, int din, int dout, int act, const float *w_f32,
                         const float *bias_f32, const char *residual_tensor);           /* :733-738 */
int wavec_add_linear_f16(void *handle, const char *name, const char *in_tensor,
                         const char *out_tensor, int din, int dout, int act,
                         const uint16_t *w_f16, const float *bias_f32,
                         const char *residual_tensor);                                  /* :740-745 */
int wavec_add_linear_bf16(void *handle, const char *name, const char *in_tensor,
                          const char *out_tensor, int din, int dout, int act,
                          const uint16_t *w_bf16, const float *bias_f32,
                          const char *residual_tensor);                                 /* :747-759 */
int wavec_add_upconv2x2(void *handle, const char *name, const char *in_tensor,
                        const char *out_tensor, int cin, int cout, const float *w_f32,
                        const float *bias_f32);                                          /* :761-771 */
int wavec_add_maxpool(void *handle, const char *name, const char *in_tensor, const char *out_tensor,
                      int k, int stride, int pad);                                      /* :773-781 */
int wavec_add_upsample2x(void *handle, const char *name, const char *in_tensor,
                         const char *out_tensor);                                        /* :783-791 */
int wavec_add_rmsnorm(void *handle, const char *name, const char *in_tensor, const char *out_tensor,
                      int dim, float eps, const float *gamma_f32, int pre_folded);     /* :793-801 */
int wavec_add_swiglu(void *handle, const char *name, const char *gate_tensor,
                     const char *up_tensor, const char *out_tensor);                     /* :803-811 */
int wavec_add_rope_gqa_attn(void *handle, const char *name, const char *q_tensor,
                            const char *k_tensor, const char *v_tensor, const char *out_tensor,
                            int h_q, int h_kv, int head_dim, float rope_theta,
                            int llama3_scaling);                                         /* :813-824 */
int wavec_add_split(void *handle, const char *name, const char *in_tensor, int num_outs,
                    const char **out_tensors);                                           /* :826-839 */
int wavec_add_slice(void *handle, const char *name, const char *in_tensor, int num_outs,
                    const char **out_tensors, const int *slice_sizes);                  /* :841-858 */
int wavec_add_concat(void *handle, const char *name, int num_ins, const char **in_tensors,
                     const char *out_tensor);                                            /* :860-873 */

/* ---- options, compile, summary, .tcff (k44_wave_executor.cu:875-954) ------------------------ */
int wavec_set_output(void *handle, const char *out_tensor);
int wavec_set_reuse_canvas(void *handle, int reuse_canvas);
int wavec_set_batch_size(void *handle, int batch_size);
int wavec_set_target_preset(void *handle, const char *preset_name);
int wavec_compile(void *handle);
/* JSON owned by the handle, valid until the next compile (:923-929). */
const char *wavec_get_summary_json(void *handle);
int wavec_save_tcff(void *handle, const char *tcff_path, const char *model_prefix);
int wavec_save_tcff_ex(void *handle, const char *tcff_path, const char *model_prefix,
                       int include_canvas, int include_geometry);
int wavec_load_tcff_weights(void *handle, const char *tcff_path);

/* ---- GPU execution (k44_wave_executor.cu:956-986) ------------------------------------------- */
int wavec_gpu_init_plan(void *handle);
/* in: [c][h][w] fp32 of the plan input; out: [c][h][w] fp32 of the plan output. */
int wavec_gpu_infer_f32(void *handle, const float *h_in, int in_elems, float *h_out,
                        int out_elems, float *out_gpu_ms);

/* ================================ build extensions ========================================== */

/* Text of the last failure on the calling thread ("" if none).  No reference counterpart. */
const char *wavec_last_error(void);

/* Sparse wave: `cout` neurons, each with `fan_in` synapses; neurons [r*cluster, (r+1)*cluster)
 * share index row r.  rows: [cout/cluster][fan_in] input-channel (substrate position) indices;
 * w_f16: [cout][fan_in] fp16 bits; bias_f16: [cout] fp16 bits or NULL; act: K44_ACT_*.
 * Replaces nothing in the reference: its builders only emit dense rows
 * (k44_wave_compiler.hpp:692-807). */
int wavec_add_sparse_wave(void *handle, const char *name, const char *in_tensor,
                          const char *out_tensor, int cout, int fan_in, int cluster,
                          const uint32_t *rows, const uint16_t *w_f16, const uint16_t *bias_f16,
                          int act, const char *residual_tensor);

/* Dendritic-cluster form: row r = K segments of S consecutive input channels starting at
 * starts[r*K + k]; w_f16: [cout][K*S]. */
int wavec_add_cluster_wave(void *handle, const char *name, const char *in_tensor,
                           const char *out_tensor, int cout, int K, int S, int cluster,
                           const uint32_t *starts, const uint16_t *w_f16, const uint16_t *bias_f16,
                           int act, const char *residual_tensor);

/* Pruned projection: neuron j keeps its own K clusters of S consecutive input channels starting
 * at starts[j*K + k]; w_f16: [cout][K*S] in the same cluster order.  Compiled to pattern-sorted
 * tiles of `tile` neurons (one sub-wave per cluster-union size, outputs restored through
 * cout_map, epilogue y = act(v + r)); cout < 65535. */
int wavec_add_pruned_wave(void *handle, const char *name, const char *in_tensor,
                          const char *out_tensor, int cout, int K, int S, int tile,
                          const uint32_t *starts, const uint16_t *w_f16, const uint16_t *bias_f16,
                          int act, const char *residual_tensor);

/* Fills the plan input on the device with the synthetic substrate
 * x(pos, t) = fp16_rne((int32(h >> 40) - 2^23) * 2^-23),
 * h = splitmix64(((pos << 20) | t) ^ splitmix64(seed)); padding tokens are 0. */
int wavec_gpu_fill_input_uniform(void *handle, unsigned long long seed);

/* Runs the whole plan `iters` times on the executor stream; average ms per run (HIP events).
 * With tuning program=1, decode-sized plans (every run a narrow projection, decode RMSNorm +
 * token shift, embedding or argmax) run each execution as one persistent launch whose stages
 * wait on device-scope completion counters (kernels/k44_program.hpp); a stage wait past its
 * limit (tuning prog_spin_ms) ends that launch early and this call (or the next
 * wavec_gpu_sync) returns -1 naming the stage.  The report's "program" says whether a plan
 * takes it and why not. */
int wavec_gpu_execute(void *handle, int iters, float *out_ms_per_iter);
int wavec_gpu_sync(void *handle);
/* Per-item timestamps of the last persistent launch of a plan initialised with tuning
 * prog_trace=1: 8 words per work item in stage order (item start, wait released, completion
 * signalled, in ticks of the 100 MHz device real-time counter; the workgroup that ran it;
 * projection items: inputs arrived, MFMAs done; stores performed).  No reference counterpart
 * (a measurement aid). */
int wavec_gpu_program_trace(void *handle, unsigned long long *dst, unsigned long long n_words);
/* Runs plan commands [first_cmd, first_cmd + n_cmds) kernel by kernel and waits for them: lets a
 * caller inspect every intermediate tensor before the canvas allocator reuses its memory. */
int wavec_gpu_execute_range(void *handle, int first_cmd, int n_cmds);

/* Raw fp16 access to the canvas (element offsets / counts). */
int wavec_gpu_read_canvas(void *handle, unsigned long long elem_off, unsigned long long n_elems,
                          uint16_t *dst);
int wavec_gpu_write_canvas(void *handle, unsigned long long elem_off, unsigned long long n_elems,
                           const uint16_t *src);

/* ---- 1-D token ops of LLM-shaped plans (no reference counterpart: its executor has no token
 * shift, embedding or argmax, and no decode state) -------------------------------------------- */
/* Causal depth-wise mix y[c][t] = sum_{i<rf} mu[c][i] * x[c][t-i] inside requests of seq_len
 * tokens (decode = 0, prefill), or one token per request with the rf-1 previous inputs carried in
 * a per-plan state block [dim][rf-1][64] (decode = 1).  mu_f16: [dim][rf]. */
int wavec_add_token_shift(void *handle, const char *name, const char *in_tensor,
                          const char *out_tensor, int dim, int rf, int seq_len,
                          const uint16_t *mu_f16, int decode);
/* y[c][t] = table[id[t]][c]; ids from wavec_gpu_set_ids or the previous run's argmax; tok_in is a
 * 1-D tensor that supplies the token axis.  table_f16: [vocab][dim]. */
int wavec_add_embedding(void *handle, const char *name, const char *tok_in, const char *out_tensor,
                        int vocab, int dim, const uint16_t *table_f16);
/* id[t] = argmax_c x[c][t] (lowest index on ties) into the plan's token-id buffer. */
int wavec_add_argmax(void *handle, const char *name, const char *in_tensor, const char *out_tensor);

int wavec_gpu_set_ids(void *handle, const uint32_t *ids, int n);
int wavec_gpu_get_ids(void *handle, uint32_t *ids, int n);
/* Record the argmax ids of the next `steps` plan runs (device-side counter); get_history returns
 * the number of steps recorded and copies up to n ids ([step][token]). */
int wavec_gpu_set_history(void *handle, int steps);
int wavec_gpu_get_history(void *handle, uint32_t *out, int n);
/* Replay each plan run as one captured HIP graph (enable = 1) instead of kernel by kernel. */
int wavec_gpu_use_graph(void *handle, int enable);
/* Device-to-device copies between two initialised plans (same GPU). */
int wavec_gpu_copy_canvas(void *dst_handle, unsigned long long dst_elem_off, void *src_handle,
                          unsigned long long src_elem_off, unsigned long long n_elems);
int wavec_gpu_copy_ids(void *dst_handle, int dst_first, void *src_handle, int src_first,
                       int src_step, int n);

/* ---- stand-alone kernels on caller-owned device memory (asynchronous on `stream`, a hipStream_t
 * or NULL for the null stream; pointers are device pointers) --------------------------------- */
/* Device memory for callers of the stand-alone kernels that have no allocator of their own
 * (the whitepaper benchmark allocates with hipMalloc directly).  No reference counterpart. */
void *wavec_dev_malloc(unsigned long long bytes);
int wavec_dev_free(void *p);
int wavec_dev_upload(void *dst_dev, const void *src_host, unsigned long long bytes);
int wavec_dev_download(void *dst_host, const void *src_dev, unsigned long long bytes);
int wavec_dev_synchronize(void);
/* Synthetic substrate rows pos0 .. pos0+rows-1 (the generator of wavec_gpu_fill_input_uniform) into
 * dst [rows][stride] fp16; tokens >= valid are 0.  Synchronous. */
int wavec_dev_fill_uniform(void *dst, unsigned long long rows, unsigned int stride,
                           unsigned int valid, unsigned long long pos0, unsigned long long seed);
/* HIP events on the null stream around stand-alone launches: begin, then end returns the
 * elapsed milliseconds (waits for the end event). */
int wavec_dev_time_begin(void);
int wavec_dev_time_end(float *ms);
/* Token64 wave, replaces launch_k44_f16_forward (whitepaper/sparse_wmma_kernel/kernels/
 * kernel44_immutable.cuh:285-297, kernel :200-259): X [ceil(batch/64)][Cin][64] fp16,
 * Y [ceil(batch/64)][Cout][64] fp16, cluster_indices [Cout/cluster_size][16*B_vec16] u32 input
 * positions (neurons j share row j/cluster_size), cluster_weights_wmma [Cout/16][B_vec16][32]
 * vectors of 8 fp16 (RDNA4 WMMA order, as written by convert_raw_to_wmma), neuron_bias [Cout] fp16
 * (NULL = 0).  Y[t][j][m] = fp16_rtz(bias[j] + sum_k W[j][k] X[t][idx[j/cluster][k]][m]), fp32
 * accumulation, every one of the 64 tokens of every tile.  cluster_size: a multiple of 16
 * dividing Cout.  64-bit addressing for any Cin; an index >= Cin reads as a zero row. */
int wavec_k44_f16_forward_token64(void *Y, const void *X, const uint32_t *cluster_indices,
                                  const void *cluster_weights_wmma, const void *neuron_bias,
                                  uint32_t batch_size, uint32_t Cin, uint32_t Cout,
                                  uint32_t B_vec16, uint32_t cluster_size, void *stream);
/* Stand-alone argmax over caller-owned device memory (the decode plans' ARGMAX_1D op, no
 * reference counterpart): ids[t] = the lowest channel c with the largest logits[c * stride + t]
 * (fp16), for t < tokens; logits [vocab][stride], stride a multiple of 64, tokens <= stride;
 * logits 8-byte aligned (a multiple of 4 fp16 elements from an allocation's start) and ids
 * 4-byte aligned, else -1 before any launch.
 * Two passes; the per-chunk (value, index) partials live in a workspace the library allocates
 * and frees on `stream` for the call (hipMallocAsync / hipFreeAsync).  Asynchronous. */
int wavec_argmax_f16(uint32_t *ids, const void *logits, uint32_t vocab, uint32_t stride,
                     uint32_t tokens, void *stream);
/* wavec_argmax_f16 without any allocation, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  The per-chunk partials live in a fixed 4 MiB array inside the
 * library's device code (one per GPU, held until the process ends; enough for
 * strides up to 524,288 tokens: sizes that need more return -1 with a message).  Calls that
 * overlap on one GPU share that array and race; ids, results and arguments otherwise as
 * wavec_argmax_f16. */
int wavec_argmax_f16_noalloc(uint32_t *ids, const void *logits, uint32_t vocab, uint32_t stride,
                             uint32_t tokens, void *stream);
/* GPU weight interleave, replaces interleave_weights_cluster16_wmma_gpu_kernel
 * (kernel44_immutable.cuh:261-267, kernels/rocm/kernel44_rocm_pack.cuh:285-290): row-major
 * [num_output_neurons][8*B_vec8] fp16 (vectors of 8) -> WMMA vector order; neurons % 16 == 0,
 * B_vec8 even. */
int wavec_interleave_weights_wmma(void *dst_wmma, const void *src_compact,
                                  uint32_t num_output_neurons, uint32_t B_vec8, void *stream);

/* JSON: per wave the kernel path taken and why, its segment schedule (K, S, step) and
 * accounting (flops, distinct substrate rows); per token op whether it was folded; the group
 * launches; "runs": the whole-plan schedule as lists of plan command indices.  "{}" before a
 * successful init. */
const char *wavec_gpu_exec_report_json(void *handle);

/* Runs [first_run, first_run + n_runs) of the whole-plan schedule (the "runs" of the report:
 * token ops, VALU waves and group launches, with folded multiplies and fused RMSNorm + token
 * shift exactly as wavec_gpu_execute launches them) and waits for them.  Lets a caller check the
 * whole-plan execution run by run.  No reference counterpart. */
int wavec_gpu_execute_runs(void *handle, int first_run, int n_runs);
/* Strided canvas read: `cols` elements from each of `rows` rows, row r starting at
 * elem_off + r * row_stride, packed into dst [rows][cols].  The range must lie inside the
 * canvas allocation. */
int wavec_gpu_read_canvas_2d(void *handle, unsigned long long elem_off, unsigned long long rows,
                             unsigned long long row_stride, unsigned long long cols,
                             uint16_t *dst);

/* Process-wide executor tuning switches, for A/B tests and benchmarks (no reference
 * counterpart).  Every switch is -1 (the executor's own choice) until set; a value is read when
 * a plan is initialised.  No switch changes what a plan computes.  Keys:
 *   "path" 0 VALU for every wave / 1 MFMA (init fails where no MFMA tiling exists);
 *   "dma" 0 register-staged MFMA tile instead of the LDS ring; "dma_stages" 2 | 4;
 *   "nt" 0 | 1 non-temporal gather loads; "splitk" 0 no split-K on wide MFMA waves;
 *   "lane8" 0 | 1 tokens per VALU lane 4 | 8; "ksplit" 1 | 4 waves per neuron (VALU);
 *   "stream_kernel" 0 | 1; "narrow" 0 no narrow MFMA kernel; "narrow_chunk" >= 16 k-steps;
 *   "group" 0 no group launches; "group_split" 0 groups keep their members' split-K;
 *   "fuse" 0 no folded multiplies or RMSNorm + token-shift kernels; "sort" 0 segments in
 *   index-row order; "wlds" 0 VALU weights read per batch; "t64_ring" 0 | 1 | 2 Token64
 *   per-wave kernel, 64-neuron x 4-tile or 128-neuron x 2-tile ring kernel only;
 *   "xcd_order" 0 | 1 | 2 MFMA tile kernels take work items in plain workgroup order, as
 *   contiguous ranges per XCD, or as per-wave shares of every XCD, longest waves first (the
 *   automatic choice); "narrow_wgs" >= 1 workgroups a narrow wave of 64/128-neuron tiles is
 *   split to reach (contraction chunks of >= 16 k-steps); "narrow_reduce" 0 | 1 split narrow
 *   waves of 64/128-neuron tiles reduce their partials in a second kernel / in the last
 *   workgroup of each tile (the automatic choice); "dma_prod" 0 | 1 LDS-ring MFMA waves of
 *   32/64-neuron tiles load and multiply in every wave / issue their loads from producer waves
 *   (4-stage ring); "program" 0 | 1 kernel-by-kernel (automatic) / one persistent launch per
 *   decode-sized execution; "prog_spin_ms" >= 0 that launch's wait limit; "prog_trace" 0 | 1
 *   its per-item timestamps; "narrow_pre" 0 | 1 narrow waves read their weights' address and
 *   geometry from their descriptors / from preloaded kernel arguments (automatic);
 *   "narrow_local" 0 | 1 split narrow waves reduced in the launch meet through device-coherent
 *   memory / through the L2 of the XCD every chunk of a tile runs on (automatic, where a
 *   set-up probe finds workgroups 8 apart in launch order sharing an XCD; a tile whose chunks
 *   met no one leaves its counter nonzero and makes wavec_gpu_execute fail); "narrow_byy" 0 | 1
 *   narrow group launches as 1-D grids (each workgroup's wave from the prefix sums) / as
 *   (workgroups x waves) grids where those launch at most 1.5x the work items (automatic);
 *   "embed_refresh" 0 | 1 a decode embedding never / also (automatic) refreshes the compact
 *   state copy of the first layer's folded token shift (0: that RMSNorm + shift runs alone).
 * wavec_set_tuning returns -1 (with a message) for an unknown key or a value the key does not
 * honour: -1 is always accepted; "dma_stages" takes 2 | 4, "ksplit" 1 | 4, "xcd_order" 0..2,
 * "t64_ring" 0..2, "narrow_chunk" >= 16, "narrow_wgs" >= 1, "prog_spin_ms" >= 0, every
 * other key 0 | 1.  wavec_get_tuning returns the
 * value or -2 for an unknown key. */
int wavec_set_tuning(const char *key, int value);
int wavec_get_tuning(const char *key);
void wavec_reset_tuning(void);

#ifdef __cplusplus
}
#endif
#endif /* K44WAVEC_H */
