// k44_aux.hpp — VALU kernels of the 1-D token ops around the waves (LLM-shaped plans).
//
// All tensors are channel-major on the canvas: element (c, t) at base + c*stride + t.
//  * RMSNORM_1D (reference kernels/common/kernel44_valu_pack.cuh:104-134): per token t,
//    y[c][t] = x[c][t] * rsqrt(sum_c x[c][t]^2 / D + eps) * gamma[c]   (gamma = 1 when folded).
//    Token counts below 8,192 (decode) sum the squares exactly (k44_sumsq.hpp); wide token
//    counts (prefill) sum them in fp32.
//  * SWIGLU_MUL_1D (reference :135-143): y = gate * up, element-wise (SiLU is fused into the gate
//    projection's epilogue).
//  * TOKEN_SHIFT_1D (build extension): causal depth-wise mix over the last RF tokens of the same
//    request, y[c][t] = sum_{i<RF} mu[c][i] * x[c][t-i] (x[c][t-i] = 0 before the request
//    start).  Decode mode: one token per request, the RF-1 previous inputs come from a state
//    block [c][RF-1][64] that the kernel shifts in place.  Prefill mode writes the same state
//    block (the last RF-1 inputs of every request) for the decode plan to continue from.
//  * EMBED_1D / ARGMAX_1D (build extension): y[c][t] = E[id[t]][c]; id[t] = argmax_c x[c][t]
//    (lowest index on ties), optionally also appended to a history buffer.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace k44dev {

// Token shift fused into an RMSNorm (launch_rmsnorm's `shift`): its output y2, mixing weights
// mu [D][rf], state [D][rf-1][64] (nullptr: none); tokens is filled in by the launcher.
// seq_len 0: the decode shift (one token per request); > 0: the prefill shift over requests of
// seq_len tokens (rmsnorm_shift_prefill_ok must hold).
struct RmsShift {
    __half *y2;
    const __half *mu;
    __half *state;
    uint32_t rf, tokens;
    uint32_t seq_len = 0;
};

// Shapes the fused prefill RMSNorm + token shift kernel takes: 32-token workgroups covering
// every token column (tokens == stride), D <= 2048 channels, rf 1..5 (its registers hold the 4
// tokens before each block), requests of a multiple of 8 tokens, and token counts at which the
// norm alone runs the register-resident kernel too (>= 256 workgroups), whose sums it repeats
// (so fused and separate launches give the same values).
inline bool rmsnorm_shift_prefill_ok(uint32_t D, uint32_t stride, uint32_t tokens, uint32_t rf,
                                     uint32_t seq_len) {
    return D > 0u && D <= 2048u && tokens == stride && tokens % 32u == 0u &&
           tokens / 32u >= 256u && rf >= 1u && rf <= 5u && seq_len > 0u && seq_len % 8u == 0u;
}

// slots (nullable, decode octet kernel only: at most 16 tokens, no fused prefill shift): the
// n_slots per-tile exact sums of squares of x stored by the waves that produced it (16 tokens x
// 2 words each, k44_sumsq.hpp); the kernel adds them instead of summing all D channels (the
// same scales bit for bit).
hipError_t launch_rmsnorm(__half *y, const __half *x, const __half *gamma, uint32_t D,
                          uint32_t stride, uint32_t tokens, float eps, hipStream_t stream,
                          const RmsShift *shift = nullptr, const uint64_t *slots = nullptr,
                          uint32_t n_slots = 0);
hipError_t launch_mul(__half *y, const __half *a, const __half *b, uint64_t n,
                      hipStream_t stream);
// y = fp16(a * fp16(b * c)) element-wise (a chain of two multiplies in one pass); y may be
// a, b or c exactly (each element is read before it is written, by the same thread).
hipError_t launch_mul3(__half *y, const __half *a, const __half *b, const __half *c, uint64_t n,
                       hipStream_t stream);
hipError_t launch_token_shift(__half *y, const __half *x, const __half *mu, __half *state,
                              uint32_t D, uint32_t stride, uint32_t tokens, uint32_t rf,
                              uint32_t seq_len, int decode, hipStream_t stream);
// slots (nullable; decode: at most 16 tokens, D % 64 == 0, 16-byte aligned table and output):
// every 64-channel block b of the output also stores the exact per-token sums of squares of
// the values it stored (k44_sumsq.hpp) at slots[(b * 16 + t) * 2 + 0 / 1] (limbs 0 | 1, limb 2
// | inf / NaN flags), the producer side of an RMSNorm folded into the readers of y.
// cp (with slots only): rows of 16 halves copied from src + r * sstride to dst + r * dstride
// by the same launch (a folded token shift's compact state copy, refreshed before its readers).
struct EmbedCopy {
    const __half *src = nullptr;
    __half *dst = nullptr;
    uint32_t rows = 0, sstride = 0, dstride = 0;
};
hipError_t launch_embed(__half *y, const __half *table, const uint32_t *ids, uint32_t D,
                        uint32_t vocab, uint32_t stride, uint32_t tokens, hipStream_t stream,
                        uint64_t *slots = nullptr, const EmbedCopy &cp = EmbedCopy{});
// history (nullable): ids are also stored at history[*step_ctr][t] while *step_ctr <
// hist_steps, and *step_ctr is incremented after the argmax (device-side, graph-safe).
// Two passes: per-chunk (value, index) partials in `scratch` (argmax_scratch_floats(V, stride)
// floats), then a per-token merge in chunk order.
size_t argmax_scratch_floats(uint32_t V, uint32_t stride);
hipError_t launch_argmax(uint32_t *ids, uint32_t *history, uint32_t *step_ctr,
                         uint32_t hist_steps, const __half *x, uint32_t V, uint32_t stride,
                         uint32_t tokens, float *scratch, hipStream_t stream);

// Packs `cols` elements of `rows` rows `row_stride` apart into dst [rows][cols] (16-bit words).
hipError_t launch_gather_cols(uint16_t *dst, const uint16_t *src, uint64_t rows,
                              uint64_t row_stride, uint64_t cols, hipStream_t stream);

}  // namespace k44dev
