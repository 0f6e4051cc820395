/*
 * TEST INFRASTRUCTURE — CPU oracle for the quantized GGML GEMM path.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this code, as the checker. The product (the HIP library) never links it.
 *
 * Every function restates the reference line by line; each cites the
 * reference file:line it follows. Build with -O2 -ffp-contract=off and without
 * -ffast-math so that fp32 expressions round exactly as the reference's do on
 * x86-64.
 */
#include "pfng_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "pfng_iq2xxs_grid.h"

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------- */
/* fp16 <-> fp32                                                              */
/* ------------------------------------------------------------------------- */

static inline float f32_from_bits(uint32_t b) {
    float f;
    memcpy(&f, &b, sizeof f);
    return f;
}

static inline uint32_t f32_to_bits(float f) {
    uint32_t b;
    memcpy(&b, &f, sizeof b);
    return b;
}

/* include/ggml.h:83-97 */
float pfo_fp16_to_fp32(uint16_t h) {
    const uint32_t w = (uint32_t)h << 16;
    const uint32_t sign = w & UINT32_C(0x80000000);
    const uint32_t two_w = w + w;
    const uint32_t exp_offset = UINT32_C(0xE0) << 23;
    const float exp_scale = 0x1.0p-112f;
    const float normalized = f32_from_bits((two_w >> 4) + exp_offset) * exp_scale;
    const uint32_t magic_mask = UINT32_C(126) << 23;
    const float magic_bias = 0.5f;
    const float denormalized = f32_from_bits((two_w >> 17) | magic_mask) - magic_bias;
    const uint32_t denormalized_cutoff = UINT32_C(1) << 27;
    return f32_from_bits(sign | (two_w < denormalized_cutoff ? f32_to_bits(denormalized) : f32_to_bits(normalized)));
}

/* include/ggml.h:99-117 */
uint16_t pfo_fp32_to_fp16(float value) {
    const float scale_to_inf = 0x1.0p+112f;
    const float scale_to_zero = 0x1.0p-110f;
    float base = (fabsf(value) * scale_to_inf) * scale_to_zero;
    const uint32_t w = f32_to_bits(value);
    const uint32_t shl1_w = w + w;
    const uint32_t sign = w & UINT32_C(0x80000000);
    uint32_t bias = shl1_w & UINT32_C(0xFF000000);
    if (bias < UINT32_C(0x71000000)) bias = UINT32_C(0x71000000);
    base = f32_from_bits((bias >> 1) + UINT32_C(0x07800000)) + base;
    const uint32_t bits = f32_to_bits(base);
    const uint32_t exp_bits = (bits >> 13) & UINT32_C(0x00007C00);
    const uint32_t mantissa_bits = bits & UINT32_C(0x00000FFF);
    const uint32_t nonsign = exp_bits + mantissa_bits;
    return (uint16_t)((sign >> 16) | (shl1_w > UINT32_C(0xFF000000) ? UINT16_C(0x7E00) : nonsign));
}

void pfo_fp16_to_fp32_n(const uint16_t *h, float *f, size_t n) {
    for (size_t i = 0; i < n; ++i) f[i] = pfo_fp16_to_fp32(h[i]);
}

void pfo_fp32_to_fp16_n(const float *f, uint16_t *h, size_t n) {
    for (size_t i = 0; i < n; ++i) h[i] = pfo_fp32_to_fp16(f[i]);
}

/* ------------------------------------------------------------------------- */
/* std::mt19937 (the generator of bench/framework/benchmark.cpp:41) and the   */
/* libstdc++ algorithms behind uniform_real_distribution<float> and           */
/* uniform_int_distribution<unsigned> (benchmark.cpp:30,77-79).               */
/* ------------------------------------------------------------------------- */

void pfo_mt_seed(pfo_mt19937 *g, uint32_t seed) {
    g->state[0] = seed;
    for (uint32_t i = 1; i < 624; ++i)
        g->state[i] = UINT32_C(1812433253) * (g->state[i - 1] ^ (g->state[i - 1] >> 30)) + i;
    g->index = 624;
}

static void mt_twist(pfo_mt19937 *g) {
    for (uint32_t i = 0; i < 624; ++i) {
        const uint32_t y = (g->state[i] & UINT32_C(0x80000000)) | (g->state[(i + 1) % 624] & UINT32_C(0x7fffffff));
        uint32_t v = g->state[(i + 397) % 624] ^ (y >> 1);
        if (y & 1u) v ^= UINT32_C(0x9908b0df);
        g->state[i] = v;
    }
    g->index = 0;
}

uint32_t pfo_mt_next(pfo_mt19937 *g) {
    if (g->index >= 624) mt_twist(g);
    uint32_t y = g->state[g->index++];
    y ^= y >> 11;
    y ^= (y << 7) & UINT32_C(0x9d2c5680);
    y ^= (y << 15) & UINT32_C(0xefc60000);
    y ^= y >> 18;
    return y;
}

/* generate_canonical<float, 24> over a 32-bit engine takes one draw:
 * u / 2^32 in float, clamped below 1; the distribution then returns
 * ret * (b - a) + a with separate fp32 rounding of the product and the sum. */
float pfo_uniform_real(pfo_mt19937 *g, float a, float b) {
    const float sum = (float)pfo_mt_next(g);
    const float tmp = 4294967296.0f;
    float ret = sum / tmp;
    if (ret >= 1.0f) ret = nextafterf(1.0f, 0.0f);
    const float span = b - a;
    const float scaled = ret * span;
    return scaled + a;
}

/* Downscaling by Lemire's nearly divisionless method with a 64-bit product,
 * the path libstdc++ takes when the engine range is exactly 2^32. */
uint32_t pfo_uniform_int(pfo_mt19937 *g, uint32_t a, uint32_t b) {
    const uint32_t range = b - a + 1u;
    uint64_t product = (uint64_t)pfo_mt_next(g) * (uint64_t)range;
    uint32_t low = (uint32_t)product;
    if (low < range) {
        const uint32_t threshold = (uint32_t)(0u - range) % range;
        while (low < threshold) {
            product = (uint64_t)pfo_mt_next(g) * (uint64_t)range;
            low = (uint32_t)product;
        }
    }
    return (uint32_t)(product >> 32) + a;
}

void pfo_mt_draws(uint32_t seed, uint32_t *out, size_t n) {
    pfo_mt19937 g;
    pfo_mt_seed(&g, seed);
    for (size_t i = 0; i < n; ++i) out[i] = pfo_mt_next(&g);
}

void pfo_uniform_real_draws(uint32_t seed, float a, float b, float *out, size_t n) {
    pfo_mt19937 g;
    pfo_mt_seed(&g, seed);
    for (size_t i = 0; i < n; ++i) out[i] = pfo_uniform_real(&g, a, b);
}

/* ------------------------------------------------------------------------- */
/* quantizers                                                                 */
/* ------------------------------------------------------------------------- */

/* std::max / std::min semantics: max(a,b) = (a < b) ? b : a, min(a,b) = (b < a) ? b : a */
static inline float smax(float a, float b) { return (a < b) ? b : a; }
static inline float smin(float a, float b) { return (b < a) ? b : a; }

/* llama_reference.cpp:13-36 */
void pfo_quantize_row_q4_0(const float *input, pfng_block_q4_0 *output, size_t count) {
    for (size_t block = 0; block < count / PFNG_QK4_0; ++block) {
        float absolute_max = 0.0f;
        float signed_max = 0.0f;
        for (size_t i = 0; i < PFNG_QK4_0; ++i) {
            const float value = input[block * PFNG_QK4_0 + i];
            if (absolute_max < fabsf(value)) {
                absolute_max = fabsf(value);
                signed_max = value;
            }
        }
        const float scale = signed_max / -8.0f;
        const float inverse_scale = scale != 0.0f ? 1.0f / scale : 0.0f;
        output[block].d = pfo_fp32_to_fp16(scale);
        for (size_t i = 0; i < PFNG_QK4_0 / 2; ++i) {
            const float low = input[block * PFNG_QK4_0 + i] * inverse_scale;
            const float high = input[block * PFNG_QK4_0 + PFNG_QK4_0 / 2 + i] * inverse_scale;
            const int8_t tl = (int8_t)(low + 8.5f);
            const int8_t th = (int8_t)(high + 8.5f);
            const uint8_t qlow = (uint8_t)(tl < 15 ? tl : 15);
            const uint8_t qhigh = (uint8_t)(th < 15 ? th : 15);
            output[block].qs[i] = (uint8_t)(qlow | (uint8_t)(qhigh << 4));
        }
    }
}

/* llama_reference.cpp:38-52 */
void pfo_quantize_row_q8_0(const float *input, pfng_block_q8_0 *output, size_t count) {
    for (size_t block = 0; block < count / PFNG_QK8_0; ++block) {
        float absolute_max = 0.0f;
        for (size_t i = 0; i < PFNG_QK8_0; ++i) absolute_max = smax(absolute_max, fabsf(input[block * PFNG_QK8_0 + i]));
        const float scale = absolute_max / 127.0f;
        const float inverse_scale = scale != 0.0f ? 1.0f / scale : 0.0f;
        output[block].d = pfo_fp32_to_fp16(scale);
        for (size_t i = 0; i < PFNG_QK8_0; ++i)
            output[block].qs[i] = (int8_t)roundf(input[block * PFNG_QK8_0 + i] * inverse_scale);
    }
}

/* llama_reference.cpp:54-70 */
void pfo_quantize_row_q8_K(const float *input, pfng_block_q8_K *output, size_t count) {
    for (size_t b = 0; b < count / PFNG_QK_K; ++b) {
        float amax = 0.0f;
        for (size_t i = 0; i < PFNG_QK_K; ++i) amax = smax(amax, fabsf(input[b * PFNG_QK_K + i]));
        output[b].d = amax / 127.0f;
        const float inv = output[b].d != 0.0f ? 1.0f / output[b].d : 0.0f;
        for (size_t i = 0; i < PFNG_QK_K; ++i) output[b].qs[i] = (int8_t)roundf(input[b * PFNG_QK_K + i] * inv);
        for (size_t i = 0; i < PFNG_QK_K / 16; ++i) {
            output[b].bsums[i] = 0;
            for (size_t j = 0; j < 16; ++j) output[b].bsums[i] = (int16_t)(output[b].bsums[i] + output[b].qs[i * 16 + j]);
        }
    }
}

/* llama_reference.cpp:72-111, including its packing of sub-blocks 4..7
 * (scales[i+8] carries the high 4 bits of s[i+4] and m[i+4]). */
void pfo_quantize_row_q4_K(const float *input, pfng_block_q4_K *output, size_t count) {
    for (size_t b = 0; b < count / PFNG_QK_K; ++b) {
        pfng_block_q4_K *o = &output[b];
        const float *x = input + b * PFNG_QK_K;
        float ls[8], lm[8], maxs = 0.0f, maxm = 0.0f;
        for (size_t sb = 0; sb < 8; ++sb) {
            float lo = x[sb * 32], hi = lo;
            for (size_t j = 1; j < 32; ++j) {
                const float v = x[sb * 32 + j];
                lo = smin(lo, v);
                hi = smax(hi, v);
            }
            ls[sb] = (hi - lo) / 15.0f;
            lm[sb] = -lo / (ls[sb] != 0.0f ? ls[sb] : 1.0f);
            maxs = smax(maxs, ls[sb]);
            maxm = smax(maxm, lm[sb]);
        }
        const float ds = maxs / 63.0f, dm = maxm / 63.0f;
        o->d = pfo_fp32_to_fp16(ds);
        o->dmin = pfo_fp32_to_fp16(dm);
        uint8_t s[8], m[8];
        for (size_t i = 0; i < 8; ++i) {
            const int si = (int)roundf(ls[i] / (ds != 0.0f ? ds : 1.0f));
            const int mi = (int)roundf(lm[i] / (dm != 0.0f ? dm : 1.0f));
            s[i] = (uint8_t)(si < 63 ? si : 63);
            m[i] = (uint8_t)(mi < 63 ? mi : 63);
        }
        for (size_t i = 0; i < 4; ++i) {
            o->scales[i] = (uint8_t)(s[i] | ((s[i + 4] & 3) << 6));
            o->scales[i + 4] = (uint8_t)(m[i] | ((m[i + 4] & 3) << 6));
            o->scales[i + 8] = (uint8_t)((s[i + 4] >> 2) | ((m[i + 4] >> 2) << 4));
        }
        for (size_t pair = 0; pair < 4; ++pair)
            for (size_t j = 0; j < 32; ++j) {
                const size_t lsb = pair * 2, hsb = lsb + 1;
                int low = (int)roundf(x[lsb * 32 + j] / (ls[lsb] != 0.0f ? ls[lsb] : 1.0f) + lm[lsb]);
                int high = (int)roundf(x[hsb * 32 + j] / (ls[hsb] != 0.0f ? ls[hsb] : 1.0f) + lm[hsb]);
                low = low < 0 ? 0 : (low > 15 ? 15 : low);
                high = high < 0 ? 0 : (high > 15 ? 15 : high);
                o->qs[pair * 32 + j] = (uint8_t)(low | (high << 4));
            }
    }
}

void pfo_quantize_q8_0(const float *x, pfng_block_q8_0 *y, size_t rows, size_t k) {
    for (size_t r = 0; r < rows; ++r) pfo_quantize_row_q8_0(x + r * k, y + r * (k / PFNG_QK8_0), k);
}

void pfo_quantize_q8_K(const float *x, pfng_block_q8_K *y, size_t rows, size_t k) {
    for (size_t r = 0; r < rows; ++r) pfo_quantize_row_q8_K(x + r * k, y + r * (k / PFNG_QK_K), k);
}

/* ------------------------------------------------------------------------- */
/* dots                                                                       */
/* ------------------------------------------------------------------------- */

static inline int32_t q4_0_block_isum(const pfng_block_q4_0 *w, const pfng_block_q8_0 *a) {
    int32_t integer_sum = 0;
    for (size_t i = 0; i < PFNG_QK4_0 / 2; ++i) {
        integer_sum += ((int)(w->qs[i] & 0x0f) - 8) * a->qs[i];
        integer_sum += ((int)(w->qs[i] >> 4) - 8) * a->qs[i + PFNG_QK4_0 / 2];
    }
    return integer_sum;
}

/* llama_reference.cpp:134-146 */
float pfo_dot_q4_0_q8_0(const pfng_block_q4_0 *weight, const pfng_block_q8_0 *activation, size_t blocks) {
    float sum = 0.0f;
    for (size_t block = 0; block < blocks; ++block) {
        const int32_t integer_sum = q4_0_block_isum(&weight[block], &activation[block]);
        const float t0 = (float)integer_sum * pfo_fp16_to_fp32(weight[block].d);
        const float t1 = t0 * pfo_fp16_to_fp32(activation[block].d);
        sum += t1;
    }
    return sum;
}

/* llama_reference.cpp:116-121 */
void pfo_q4_K_scales_mins(const pfng_block_q4_K *w, uint8_t scales[8], uint8_t mins[8]) {
    for (size_t i = 0; i < 4; ++i) {
        scales[i] = w->scales[i] & 63;
        scales[i + 4] = (uint8_t)((w->scales[i + 8] & 15) | ((w->scales[i] >> 6) << 4));
        mins[i] = w->scales[i + 4] & 63;
        mins[i + 4] = (uint8_t)((w->scales[i + 8] >> 4) | ((w->scales[i + 4] >> 6) << 4));
    }
}

/* llama_reference.cpp:113-132 */
float pfo_dot_q4_K_q8_K(const pfng_block_q4_K *w, const pfng_block_q8_K *a) {
    uint8_t scales[8], mins[8];
    pfo_q4_K_scales_mins(w, scales, mins);
    const float d = pfo_fp16_to_fp32(w->d);
    const float dmin = pfo_fp16_to_fp32(w->dmin);
    float sum = 0.0f;
    for (size_t sb = 0; sb < 8; ++sb)
        for (size_t j = 0; j < 32; ++j) {
            const uint8_t packed = w->qs[(sb / 2) * 32 + j];
            const int q = sb % 2 == 0 ? packed & 15 : packed >> 4;
            const float t0 = d * (float)scales[sb];
            const float t1 = t0 * (float)q;
            const float t2 = dmin * (float)mins[sb];
            const float t3 = t1 - t2;
            const float t4 = (float)a->qs[sb * 32 + j] * t3;
            sum += t4;
        }
    return a->d * sum;
}

/* kernels/common/iq2_xxs.h:25-41 with the 256-entry grid of
 * kernels/iq2_xxs-q8_K-RVV-common/ggml_min.h:69-134. */
void pfo_iq2_xxs_decode_subblock(const uint8_t *packed, int8_t values[32], int *scale) {
    uint32_t signs_and_scale;
    memcpy(&signs_and_scale, packed + 4, sizeof signs_and_scale);
    for (unsigned group = 0; group < 4; ++group) {
        const unsigned index = (signs_and_scale >> (7 * group)) & 0x7f;
        const unsigned parity = (unsigned)__builtin_parity(index);
        const uint8_t signs = (uint8_t)(index | (parity << 7));
        for (unsigned lane = 0; lane < 8; ++lane) {
            const int8_t magnitude = (int8_t)pfng_iq2xxs_grid_byte(packed[group], lane);
            values[group * 8 + lane] = (signs & (1u << lane)) ? (int8_t)-magnitude : magnitude;
        }
    }
    *scale = 2 * (int)((signs_and_scale >> 28) & 0x0f) + 1;
}

static inline int32_t iq2_xxs_isum(const pfng_block_iq2_xxs *weight, const pfng_block_q8_K *activation) {
    const uint8_t *packed = (const uint8_t *)weight->qs;
    int32_t sum = 0;
    for (size_t subblock = 0; subblock < PFNG_QK_K / 32; ++subblock) {
        int8_t values[32];
        int scale;
        pfo_iq2_xxs_decode_subblock(packed + subblock * 8, values, &scale);
        int32_t subblock_sum = 0;
        for (size_t i = 0; i < 32; ++i) subblock_sum += values[i] * activation->qs[subblock * 32 + i];
        sum += scale * subblock_sum;
    }
    return sum;
}

/* llama_reference.cpp:148-161 */
float pfo_dot_iq2_xxs_q8_K(const pfng_block_iq2_xxs *weight, const pfng_block_q8_K *activation) {
    const int32_t sum = iq2_xxs_isum(weight, activation);
    const float t0 = 0.125f * pfo_fp16_to_fp32(weight->d);
    const float t1 = t0 * activation->d;
    return t1 * (float)sum;
}

/* ------------------------------------------------------------------------- */
/* integer block sums                                                         */
/* ------------------------------------------------------------------------- */

void pfo_isums_q4_0_q8_0(const pfng_block_q4_0 *w, const pfng_block_q8_0 *a, size_t m, size_t n, size_t k,
                         int32_t *out) {
    const size_t nb = k / PFNG_QK4_0;
#pragma omp parallel for schedule(static)
    for (long long mi = 0; mi < (long long)m; ++mi)
        for (size_t ni = 0; ni < n; ++ni)
            for (size_t b = 0; b < nb; ++b)
                out[((size_t)mi * n + ni) * nb + b] = q4_0_block_isum(&w[ni * nb + b], &a[(size_t)mi * nb + b]);
}

void pfo_isums_q4_K_q8_K(const pfng_block_q4_K *w, const pfng_block_q8_K *a, size_t m, size_t n, size_t k,
                         int32_t *out2) {
    const size_t nb = k / PFNG_QK_K;
#pragma omp parallel for schedule(static)
    for (long long mi = 0; mi < (long long)m; ++mi)
        for (size_t ni = 0; ni < n; ++ni)
            for (size_t b = 0; b < nb; ++b) {
                const pfng_block_q4_K *wb = &w[ni * nb + b];
                const pfng_block_q8_K *ab = &a[(size_t)mi * nb + b];
                uint8_t sc[8], mn[8];
                pfo_q4_K_scales_mins(wb, sc, mn);
                int32_t isc = 0, imn = 0;
                for (size_t sb = 0; sb < 8; ++sb) {
                    int32_t s = 0;
                    for (size_t j = 0; j < 32; ++j) {
                        const uint8_t packed = wb->qs[(sb / 2) * 32 + j];
                        const int q = sb % 2 == 0 ? packed & 15 : packed >> 4;
                        s += q * ab->qs[sb * 32 + j];
                    }
                    isc += sc[sb] * s;
                    imn += mn[sb] * (ab->bsums[2 * sb] + ab->bsums[2 * sb + 1]);
                }
                out2[(((size_t)mi * n + ni) * nb + b) * 2 + 0] = isc;
                out2[(((size_t)mi * n + ni) * nb + b) * 2 + 1] = imn;
            }
}

void pfo_isums_iq2_xxs_q8_K(const pfng_block_iq2_xxs *w, const pfng_block_q8_K *a, size_t m, size_t n, size_t k,
                            int32_t *out) {
    const size_t nb = k / PFNG_QK_K;
#pragma omp parallel for schedule(static)
    for (long long mi = 0; mi < (long long)m; ++mi)
        for (size_t ni = 0; ni < n; ++ni)
            for (size_t b = 0; b < nb; ++b)
                out[((size_t)mi * n + ni) * nb + b] = iq2_xxs_isum(&w[ni * nb + b], &a[(size_t)mi * nb + b]);
}

/* ------------------------------------------------------------------------- */
/* GEMM drivers                                                               */
/* ------------------------------------------------------------------------- */

static void set_threads(int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
}

/* llama_reference.cpp:172-175, 185-189, 199-203 (loops over m, n, blocks) */
int pfo_matmul(int type, const void *weight, const void *act_q, float *out, size_t m, size_t n, size_t k,
               int threads) {
    set_threads(threads);
    if (type == PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0) {
        if (k % PFNG_QK4_0) return -1;
        const size_t nb = k / PFNG_QK4_0;
        const pfng_block_q4_0 *w = (const pfng_block_q4_0 *)weight;
        const pfng_block_q8_0 *a = (const pfng_block_q8_0 *)act_q;
#pragma omp parallel for schedule(static)
        for (long long mi = 0; mi < (long long)m; ++mi)
            for (size_t ni = 0; ni < n; ++ni)
                out[(size_t)mi * n + ni] = pfo_dot_q4_0_q8_0(w + ni * nb, a + (size_t)mi * nb, nb);
        return 0;
    }
    if (type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K || type == PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K) {
        if (k % PFNG_QK_K) return -1;
        const size_t nb = k / PFNG_QK_K;
        const pfng_block_q8_K *a = (const pfng_block_q8_K *)act_q;
#pragma omp parallel for schedule(static)
        for (long long mi = 0; mi < (long long)m; ++mi)
            for (size_t ni = 0; ni < n; ++ni) {
                float acc = 0.0f;
                for (size_t b = 0; b < nb; ++b) {
                    if (type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K)
                        acc += pfo_dot_q4_K_q8_K((const pfng_block_q4_K *)weight + ni * nb + b, a + (size_t)mi * nb + b);
                    else
                        acc += pfo_dot_iq2_xxs_q8_K((const pfng_block_iq2_xxs *)weight + ni * nb + b,
                                                    a + (size_t)mi * nb + b);
                }
                out[(size_t)mi * n + ni] = acc;
            }
        return 0;
    }
    return -2;
}

/* llama_reference.cpp:165-215: quantize activations row by row, then the GEMM. */
int pfo_compute(int type, const float *activation, const void *weight, float *out, size_t m, size_t n, size_t k,
                int threads) {
    if (type == PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0) {
        if (k % PFNG_QK8_0) return -1;
        pfng_block_q8_0 *a = (pfng_block_q8_0 *)malloc(m * (k / PFNG_QK8_0) * sizeof *a);
        if (!a) return -3;
        pfo_quantize_q8_0(activation, a, m, k);
        const int rc = pfo_matmul(type, weight, a, out, m, n, k, threads);
        free(a);
        return rc;
    }
    if (type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K || type == PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K) {
        if (k % PFNG_QK_K) return -1;
        pfng_block_q8_K *a = (pfng_block_q8_K *)malloc(m * (k / PFNG_QK_K) * sizeof *a);
        if (!a) return -3;
        pfo_quantize_q8_K(activation, a, m, k);
        const int rc = pfo_matmul(type, weight, a, out, m, n, k, threads);
        free(a);
        return rc;
    }
    return -2;
}

/* ------------------------------------------------------------------------- */
/* tolerance model                                                            */
/* ------------------------------------------------------------------------- */

int pfo_abs_terms(int type, const void *weight, const void *act_q, double *abs_terms, size_t m, size_t n,
                  size_t k, int threads) {
    set_threads(threads);
    if (type == PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0) {
        const size_t nb = k / PFNG_QK4_0;
        const pfng_block_q4_0 *w = (const pfng_block_q4_0 *)weight;
        const pfng_block_q8_0 *a = (const pfng_block_q8_0 *)act_q;
#pragma omp parallel for schedule(static)
        for (long long mi = 0; mi < (long long)m; ++mi)
            for (size_t ni = 0; ni < n; ++ni) {
                double s = 0.0;
                for (size_t b = 0; b < nb; ++b) {
                    const double t = (double)q4_0_block_isum(&w[ni * nb + b], &a[(size_t)mi * nb + b]) *
                                     (double)pfo_fp16_to_fp32(w[ni * nb + b].d) *
                                     (double)pfo_fp16_to_fp32(a[(size_t)mi * nb + b].d);
                    s += fabs(t);
                }
                abs_terms[(size_t)mi * n + ni] = s;
            }
        return 0;
    }
    if (type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K) {
        const size_t nb = k / PFNG_QK_K;
        const pfng_block_q4_K *w = (const pfng_block_q4_K *)weight;
        const pfng_block_q8_K *a = (const pfng_block_q8_K *)act_q;
#pragma omp parallel for schedule(static)
        for (long long mi = 0; mi < (long long)m; ++mi)
            for (size_t ni = 0; ni < n; ++ni) {
                double s = 0.0;
                for (size_t b = 0; b < nb; ++b) {
                    const pfng_block_q4_K *wb = &w[ni * nb + b];
                    const pfng_block_q8_K *ab = &a[(size_t)mi * nb + b];
                    uint8_t sc[8], mn[8];
                    pfo_q4_K_scales_mins(wb, sc, mn);
                    const double d = pfo_fp16_to_fp32(wb->d), dmin = pfo_fp16_to_fp32(wb->dmin);
                    for (size_t sb = 0; sb < 8; ++sb)
                        for (size_t j = 0; j < 32; ++j) {
                            const uint8_t packed = wb->qs[(sb / 2) * 32 + j];
                            const int q = sb % 2 == 0 ? packed & 15 : packed >> 4;
                            const double av = fabs((double)ab->d * (double)ab->qs[sb * 32 + j]);
                            s += av * (fabs(d * sc[sb] * q) + fabs(dmin * mn[sb]));
                        }
                }
                abs_terms[(size_t)mi * n + ni] = s;
            }
        return 0;
    }
    if (type == PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K) {
        const size_t nb = k / PFNG_QK_K;
        const pfng_block_iq2_xxs *w = (const pfng_block_iq2_xxs *)weight;
        const pfng_block_q8_K *a = (const pfng_block_q8_K *)act_q;
#pragma omp parallel for schedule(static)
        for (long long mi = 0; mi < (long long)m; ++mi)
            for (size_t ni = 0; ni < n; ++ni) {
                double s = 0.0;
                for (size_t b = 0; b < nb; ++b) {
                    const double t = 0.125 * (double)pfo_fp16_to_fp32(w[ni * nb + b].d) *
                                     (double)a[(size_t)mi * nb + b].d *
                                     (double)iq2_xxs_isum(&w[ni * nb + b], &a[(size_t)mi * nb + b]);
                    s += fabs(t);
                }
                abs_terms[(size_t)mi * n + ni] = s;
            }
        return 0;
    }
    return -2;
}

/* ------------------------------------------------------------------------- */
/* seeded input generation                                                    */
/* ------------------------------------------------------------------------- */

/* benchmark.cpp:29-32 */
static void fill_random(float *values, size_t count, pfo_mt19937 *g) {
    for (size_t i = 0; i < count; ++i) values[i] = pfo_uniform_real(g, -1.0f, 1.0f);
}

/* benchmark.cpp:34-50, 52-66, 68-94 */
int pfo_create_input(int type, int variant, uint32_t seed, size_t m, size_t n, size_t k, float *activation,
                     void *weight) {
    pfo_mt19937 g;
    pfo_mt_seed(&g, seed);
    if (type == PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0 || type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K) {
        const size_t qk = type == PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0 ? PFNG_QK4_0 : PFNG_QK_K;
        if (k % qk) return -1;
        float *wf = (float *)malloc(n * k * sizeof *wf);
        if (!wf) return -3;
        fill_random(activation, m * k, &g);
        fill_random(wf, n * k, &g);
        for (size_t r = 0; r < n; ++r) {
            if (type == PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0)
                pfo_quantize_row_q4_0(wf + r * k, (pfng_block_q4_0 *)weight + r * (k / qk), k);
            else
                pfo_quantize_row_q4_K(wf + r * k, (pfng_block_q4_K *)weight + r * (k / qk), k);
        }
        free(wf);
        return 0;
    }
    if (type == PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K) {
        if (k % PFNG_QK_K) return -1;
        fill_random(activation, m * k, &g);
        const uint32_t grid_hi = variant == 0 ? 31u : 255u;
        const float d_lo = variant == 0 ? 0.002f : 0.001f;
        const float d_hi = variant == 0 ? 0.02f : 0.01f;
        pfng_block_iq2_xxs *blocks = (pfng_block_iq2_xxs *)weight;
        const size_t count = n * (k / PFNG_QK_K);
        for (size_t i = 0; i < count; ++i) {
            blocks[i].d = pfo_fp32_to_fp16(pfo_uniform_real(&g, d_lo, d_hi));
            uint8_t *packed = (uint8_t *)blocks[i].qs;
            for (size_t sb = 0; sb < PFNG_QK_K / 32; ++sb) {
                for (size_t group = 0; group < 4; ++group) packed[sb * 8 + group] = (uint8_t)pfo_uniform_int(&g, 0, grid_hi);
                uint32_t signs_and_scale = pfo_uniform_int(&g, 0, 255) & 0x7f;
                signs_and_scale |= (pfo_uniform_int(&g, 0, 255) & 0x7f) << 7;
                signs_and_scale |= (pfo_uniform_int(&g, 0, 255) & 0x7f) << 14;
                signs_and_scale |= (pfo_uniform_int(&g, 0, 255) & 0x7f) << 21;
                signs_and_scale |= (pfo_uniform_int(&g, 0, 255) & 0x0f) << 28;
                memcpy(packed + sb * 8 + 4, &signs_and_scale, sizeof signs_and_scale);
            }
        }
        return 0;
    }
    return -2;
}

double pfo_checksum(const float *out, size_t count) {
    double sum = 0.0;
    for (size_t i = 0; i < count; i += 257) sum += out[i];
    return sum;
}
