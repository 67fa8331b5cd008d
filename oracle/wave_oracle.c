/*
 * wave_oracle.c — CPU ORACLE for the SNNtome wave hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (snntome_amd/, include/) links, loads or
 * calls this file.  It is used by tests/, by __graft_entry__.smoke() as the checker, and by
 * bench.py's cpu_baseline leg as the timed CPU path.  It is a plain-C restatement, written from
 * the documented semantics of the reference; each function cites the reference lines it
 * follows (paths relative to the reference repository root).
 *
 * Contents
 *   orc_f32_to_f16 / orc_f16_to_f32 / orc_bf16_to_f32   wavec/k44_plan_types.hpp:21-94
 *   orc_fnv1a64                                          wavec/k44_tcff_io.hpp:10-17
 *   orc_raw_to_wmma / orc_wmma_to_raw                    wavec/k44_plan_types.hpp:363-394
 *   orc_splitmix64 / orc_substrate_f16                   synthetic-data generator (own spec)
 *   orc_act                                              kernels/rocm/kernel44_rocm_pack.cuh:79-84
 *                                                        (+ GELU, erf form, id 5: build extension)
 *   orc_wave_f64      fp64-accumulate scalar wave     = stage 2 of
 *                     whitepaper/sparse_wmma_kernel/tests/error_collapse_test.cpp:104-111,
 *                     epilogue order of kernel44_rocm_pack.cuh:219-236
 *   orc_wave_f32_omp  OpenMP fp32 wave writing fp16 (RNE) into a canvas: the timed CPU baseline
 *
 * Wave semantics (one K44_WAVE command on a 1-D token canvas, kernel44_rocm_pack.cuh:145-237):
 *   row(j)    = j / cluster                      (neurons sharing one index row)
 *   v[j][m]   = bias[j] + sum_{k<K} sum_{s<S} W[j][k*S+s] * X[seg[row(j)][k] + s*step + m]
 *   out_j     = cmap ? cmap[j] : j
 *   r         = residual ? R[res_off + out_j*out_stride + m] : 0
 *   y[j][m]   = cmap ? act(v + r) : act(v) + r
 *   stored at canvas[y_off + out_j*out_stride + m], rounded to fp16 with round-half-even.
 * A reference per-synapse index row (h_idx) is the special case S = 1, K = B_raw.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#if defined(__F16C__) && defined(__AVX2__) && defined(__FMA__)
#include <immintrin.h>
#define ORC_HAVE_F16C 1
#endif

/* ---------------------------------------------------------------------------------------------
 * IEEE binary16 conversion, round-half-even; NaN -> sign | 0x7c00 | (mant >> 13) | 1
 * (wavec/k44_plan_types.hpp:21-60).  Written as a bit-level restatement.
 * ------------------------------------------------------------------------------------------- */
uint16_t orc_f32_to_f16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) {
        if (a == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7c00u | ((a & 0x7fffffu) >> 13) | 1u);
    }
    if (a < 0x38800000u) { /* |f| < 2^-14: half subnormal or zero */
        if (a < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to zero */
        uint32_t e = a >> 23;                        /* biased f32 exponent, 102..112 */
        uint32_t m = (a & 0x7fffffu) | 0x800000u;
        uint32_t sh = 126u - e;                      /* value / 2^-24 = m >> sh */
        uint32_t q = m >> sh;
        uint32_t rem = m & ((1u << sh) - 1u);
        uint32_t half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t b = a - 0x38000000u; /* rebias 127 -> 15 */
    uint32_t q = b >> 13;
    uint32_t rem = b & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    if (q >= 0x7c00u) q = 0x7c00u;
    return (uint16_t)(sign | q);
}

/* Same conversion taking the float's bit pattern (keeps signalling-NaN payloads intact). */
uint16_t orc_f32bits_to_f16(uint32_t bits) {
    float f;
    memcpy(&f, &bits, 4);
    return orc_f32_to_f16(f);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t u;
    if (e == 0x1fu) {
        u = sign | 0x7f800000u | (m << 13);
    } else if (e != 0u) {
        u = sign | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0u) {
        u = sign;
    } else { /* subnormal: m * 2^-24 */
        float v = (float)m * (1.0f / 16777216.0f);
        memcpy(&u, &v, 4);
        u |= sign;
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float orc_bf16_to_f32(uint16_t b) { /* k44_plan_types.hpp:89-94 */
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* FNV-1a 64-bit (k44_tcff_io.hpp:10-17; published offset basis / prime). */
uint64_t orc_fnv1a64(const uint8_t *p, size_t n) {
    uint64_t h = 14695981039346656037ULL;
    for (size_t i = 0; i < n; ++i) {
        h ^= p[i];
        h *= 1099511628211ULL;
    }
    return h;
}

/* ---------------------------------------------------------------------------------------------
 * RDNA4 WMMA weight order (k44_plan_types.hpp:349-375): the 16-byte vector (8 fp16) at position
 * g = (rb * B/16 + kb) * 32 + l holds W[16*rb + (l & 15)][16*kb + 8*(l >> 4) .. +8].
 * Operates on fp16 element arrays of shape [cout_pad][B].
 * ------------------------------------------------------------------------------------------- */
void orc_raw_to_wmma(uint16_t *dst, const uint16_t *src, uint32_t cout_pad, uint32_t B) {
    uint32_t kb_n = B / 16u;
    for (uint32_t rb = 0; rb < cout_pad / 16u; ++rb)
        for (uint32_t kb = 0; kb < kb_n; ++kb)
            for (uint32_t l = 0; l < 32u; ++l) {
                size_t g = ((size_t)rb * kb_n + kb) * 32u + l;
                size_t row = 16u * rb + (l & 15u);
                size_t col = 16u * kb + 8u * (l >> 4);
                memcpy(dst + g * 8u, src + row * B + col, 16);
            }
}

void orc_wmma_to_raw(uint16_t *dst, const uint16_t *src, uint32_t cout_pad, uint32_t B) {
    uint32_t kb_n = B / 16u;
    for (uint32_t rb = 0; rb < cout_pad / 16u; ++rb)
        for (uint32_t kb = 0; kb < kb_n; ++kb)
            for (uint32_t l = 0; l < 32u; ++l) {
                size_t g = ((size_t)rb * kb_n + kb) * 32u + l;
                size_t row = 16u * rb + (l & 15u);
                size_t col = 16u * kb + 8u * (l >> 4);
                memcpy(dst + row * B + col, src + g * 8u, 16);
            }
}

/* ---------------------------------------------------------------------------------------------
 * Synthetic substrate generator (the build's own specification, shared by the product's device
 * fill kernel and its numpy generator; pinned here by the SplitMix64 published known answers).
 *   sm64(x)  = SplitMix64 output for state x (state advanced once by 0x9e3779b97f4a7c15)
 *   h        = sm64(((pos << 20) | tok) ^ sm64(seed))
 *   x(pos,t) = fp16_rne( (int32(h >> 40) - 2^23) * 2^-23 )        in [-1, 1)
 * ------------------------------------------------------------------------------------------- */
uint64_t orc_splitmix64(uint64_t x) {
    uint64_t z = x + 0x9e3779b97f4a7c15ULL;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

uint16_t orc_substrate_f16(uint64_t seed, uint64_t pos, uint32_t tok) {
    uint64_t h = orc_splitmix64(((pos << 20) | (uint64_t)tok) ^ orc_splitmix64(seed));
    int32_t q = (int32_t)(h >> 40) - 8388608;
    return orc_f32_to_f16((float)q * (1.0f / 8388608.0f));
}

/* Fills rows [pos0, pos0 + npos) of a [pos][stride] fp16 substrate, tokens [0, tokens). */
void orc_fill_substrate(uint16_t *dst, uint64_t seed, uint64_t pos0, uint64_t npos,
                        uint32_t tokens, uint64_t stride) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)npos; ++i)
        for (uint32_t t = 0; t < tokens; ++t)
            dst[(uint64_t)i * stride + t] = orc_substrate_f16(seed, pos0 + (uint64_t)i, t);
}

/* Fills n_seg segments of S rows each: dst row (i*S + s) = substrate row starts[i] + s. */
void orc_fill_segments(uint16_t *dst, uint64_t seed, const uint64_t *starts, uint64_t n_seg,
                       uint32_t S, uint32_t tokens, uint64_t stride) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n_seg; ++i)
        for (uint32_t s = 0; s < S; ++s)
            for (uint32_t t = 0; t < tokens; ++t)
                dst[((uint64_t)i * S + s) * stride + t] = orc_substrate_f16(seed, starts[i] + s, t);
}

/* ---------------------------------------------------------------------------------------------
 * Activations (kernel44_rocm_pack.cuh:79-84); id 5 = GELU, 0.5 v (1 + erf(v / sqrt 2)).
 * ------------------------------------------------------------------------------------------- */
double orc_act(double v, int act) {
    switch (act) {
    case 1: return v > 0.0 ? v : 0.0;
    case 2: return 1.0 / (1.0 + exp(-v));
    case 3: return v / (1.0 + exp(-v));
    case 4: return v > 0.1 * v ? v : 0.1 * v;
    case 5: return 0.5 * v * (1.0 + erf(v * 0.70710678118654752440));
    default: return v;
    }
}

static float orc_act_f32(float v, int act) {
    switch (act) {
    case 1: return v > 0.0f ? v : 0.0f;
    case 2: return 1.0f / (1.0f + expf(-v));
    case 3: return v / (1.0f + expf(-v));
    case 4: return v > 0.1f * v ? v : 0.1f * v;
    case 5: return 0.5f * v * (1.0f + erff(v * 0.70710678f));
    default: return v;
    }
}

/* ---------------------------------------------------------------------------------------------
 * fp64 oracle (stage 2 of error_collapse_test.cpp:104-111: fp16-quantised operands summed in
 * fp64), with the epilogue of kernel44_rocm_pack.cuh:219-236.
 *   canvas   fp16 canvas (X, and R when has_residual)
 *   seg      [cout/cluster][K] element offsets into canvas of each segment start
 *   w        [cout][K*S] fp16, bias [cout] fp16 (NULL = no bias), cmap [cout] (NULL = identity)
 *   sel      neuron indices to evaluate (n_sel of them); out [n_sel][tokens] fp64, pre-rounding.
 * Returns 0.
 * ------------------------------------------------------------------------------------------- */
/* Every fp16 bit pattern as a double (orc_f16_to_f32 widened; exact). */
static double g_f16_f64[65536];
static int g_f16_f64_ready = 0;

static void f16_table_init(void) {
    if (g_f16_f64_ready) return;
    for (uint32_t h = 0; h < 65536u; ++h) g_f16_f64[h] = (double)orc_f16_to_f32((uint16_t)h);
    g_f16_f64_ready = 1;
}

int orc_wave_f64(const uint16_t *canvas, const uint64_t *seg, const uint16_t *w,
                 const uint16_t *bias, const uint16_t *cmap, uint32_t K, uint32_t S,
                 uint32_t cluster, uint64_t step, uint32_t tokens, uint64_t out_stride,
                 int act, int has_residual, uint64_t res_off, const uint32_t *sel,
                 uint32_t n_sel, double *out) {
    const uint64_t KS = (uint64_t)K * S;
    const double *tab = g_f16_f64;
    f16_table_init();
    /* Per neuron and token: acc = bias, then + w*x over k (outer) and s (inner), in that order;
     * the token loop is innermost so that a whole row of X is consumed per synapse. */
#pragma omp parallel for schedule(dynamic, 4)
    for (int64_t q = 0; q < (int64_t)n_sel; ++q) {
        uint32_t j = sel[q];
        const uint64_t *rs = seg + (uint64_t)(j / cluster) * K;
        const uint16_t *wj = w + (uint64_t)j * KS;
        double b = bias ? tab[bias[j]] : 0.0;
        uint64_t oj = cmap ? cmap[j] : j;
        double *acc = out + (uint64_t)q * tokens;
        for (uint32_t m = 0; m < tokens; ++m) acc[m] = b;
        for (uint32_t k = 0; k < K; ++k)
            for (uint32_t s = 0; s < S; ++s) {
                const double wv = tab[wj[(uint64_t)k * S + s]];
                const uint16_t *xr = canvas + rs[k] + (uint64_t)s * step;
                for (uint32_t m = 0; m < tokens; ++m) acc[m] += wv * tab[xr[m]];
            }
        for (uint32_t m = 0; m < tokens; ++m) {
            double r = has_residual ? tab[canvas[res_off + oj * out_stride + m]] : 0.0;
            acc[m] = cmap ? orc_act(acc[m] + r, act) : orc_act(acc[m], act) + r;
        }
    }
    return 0;
}

/* ---------------------------------------------------------------------------------------------
 * OpenMP fp32 path (the timed CPU baseline): every neuron j in [0, cout), fp32 accumulation,
 * result stored as fp16 (RNE) at canvas[y_off + out_j*out_stride + m].  Gathered rows are
 * streamed token-contiguously so the inner loop vectorises.  Uses up to `threads` threads
 * (0 = OpenMP default).  Returns the number of threads used.
 * ------------------------------------------------------------------------------------------- */
int orc_wave_f32_omp(uint16_t *canvas, const uint64_t *seg, const uint16_t *w,
                     const uint16_t *bias, const uint16_t *cmap, uint32_t cout, uint32_t K,
                     uint32_t S, uint32_t cluster, uint64_t step, uint32_t tokens,
                     uint64_t out_stride, int act, int has_residual, uint64_t res_off,
                     uint64_t y_off, int threads) {
    const uint64_t KS = (uint64_t)K * S;
    int used = 1;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#endif
#pragma omp parallel
    {
#ifdef _OPENMP
#pragma omp single
        used = omp_get_num_threads();
#endif
        float *acc = (float *)__builtin_alloca(sizeof(float) * tokens);
#pragma omp for schedule(dynamic, 8)
        for (int64_t jj = 0; jj < (int64_t)cout; ++jj) {
            uint32_t j = (uint32_t)jj;
            const uint64_t *rs = seg + (uint64_t)(j / cluster) * K;
            const uint16_t *wj = w + (uint64_t)j * KS;
            float b = bias ? orc_f16_to_f32(bias[j]) : 0.0f;
            for (uint32_t m = 0; m < tokens; ++m) acc[m] = b;
            for (uint32_t k = 0; k < K; ++k)
                for (uint32_t s = 0; s < S; ++s) {
                    float wv = orc_f16_to_f32(wj[(uint64_t)k * S + s]);
                    const uint16_t *xr = canvas + rs[k] + (uint64_t)s * step;
                    uint32_t m = 0;
#ifdef ORC_HAVE_F16C
                    const __m256 wv8 = _mm256_set1_ps(wv);
                    for (; m + 8u <= tokens; m += 8u) {
                        __m256 x8 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(xr + m)));
                        _mm256_storeu_ps(acc + m,
                                         _mm256_fmadd_ps(wv8, x8, _mm256_loadu_ps(acc + m)));
                    }
#endif
                    for (; m < tokens; ++m) acc[m] += wv * orc_f16_to_f32(xr[m]);
                }
            uint64_t oj = cmap ? cmap[j] : j;
            for (uint32_t m = 0; m < tokens; ++m) {
                float r = has_residual ? orc_f16_to_f32(canvas[res_off + oj * out_stride + m])
                                       : 0.0f;
                float y = cmap ? orc_act_f32(acc[m] + r, act) : orc_act_f32(acc[m], act) + r;
                canvas[y_off + oj * out_stride + m] = orc_f32_to_f16(y);
            }
        }
    }
    return used;
}
