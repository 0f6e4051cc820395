// Synthetic inputs and host weight quantizers of the benchmark harness
// (bench/framework/benchmark.cpp:29-94, bench/llama_reference/llama_reference.cpp:13-36,72-111).
//
// The generator is the C++ standard library's own std::mt19937 with
// uniform_real_distribution<float> / uniform_int_distribution<unsigned>, called
// in the reference's order, so the same (seed, shape) gives the same bytes as
// the reference harness built with the same standard library. Compiled with
// -ffp-contract=off: every fp32 step is rounded on its own, as in the
// reference's scalar code.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <random>
#include <vector>

#include "pfng_blocks.h"
#include "pfng_host.h"

namespace {

uint32_t bits_of(float f) {
    uint32_t u;
    std::memcpy(&u, &f, sizeof u);
    return u;
}
float float_of(uint32_t u) {
    float f;
    std::memcpy(&f, &u, sizeof f);
    return f;
}

// include/ggml.h:99-117: round-to-nearest-even through fp32 arithmetic.
uint16_t to_fp16(float value) {
    const float scale_to_inf = 0x1.0p+112f;
    const float scale_to_zero = 0x1.0p-110f;
    float base = (std::fabs(value) * scale_to_inf) * scale_to_zero;
    const uint32_t w = bits_of(value);
    const uint32_t shl1_w = w + w;
    const uint32_t sign = w & 0x80000000u;
    uint32_t bias = shl1_w & 0xFF000000u;
    if (bias < 0x71000000u) bias = 0x71000000u;
    base = float_of((bias >> 1) + 0x07800000u) + base;
    const uint32_t bits = bits_of(base);
    const uint32_t nonsign = ((bits >> 13) & 0x00007C00u) + (bits & 0x00000FFFu);
    return (uint16_t)((sign >> 16) | (shl1_w > 0xFF000000u ? 0x7E00u : nonsign));
}

// include/ggml.h:83-97
float from_fp16(uint16_t h) {
    const uint32_t w = (uint32_t)h << 16;
    const uint32_t sign = w & 0x80000000u;
    const uint32_t two_w = w + w;
    const float normalized = float_of((two_w >> 4) + (0xE0u << 23)) * 0x1.0p-112f;
    const float denormalized = float_of((two_w >> 17) | (126u << 23)) - 0.5f;
    return float_of(sign | (two_w < (1u << 27) ? bits_of(denormalized) : bits_of(normalized)));
}

// llama_reference.cpp:13-36: scale = (value of largest magnitude) / -8, codes
// truncated from x/scale + 8.5 and capped at 15.
void quantize_q4_0_row(const float *x, pfng_block_q4_0 *y, size_t k) {
    for (size_t b = 0; b < k / PFNG_QK4_0; ++b) {
        const float *v = x + b * PFNG_QK4_0;
        float amax = 0.0f, smax = 0.0f;
        for (size_t i = 0; i < PFNG_QK4_0; ++i)
            if (amax < std::fabs(v[i])) {
                amax = std::fabs(v[i]);
                smax = v[i];
            }
        const float d = smax / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[b].d = to_fp16(d);
        for (size_t i = 0; i < PFNG_QK4_0 / 2; ++i) {
            const int lo = std::min<int>(15, (int8_t)(v[i] * id + 8.5f));
            const int hi = std::min<int>(15, (int8_t)(v[i + PFNG_QK4_0 / 2] * id + 8.5f));
            y[b].qs[i] = (uint8_t)(lo | (hi << 4));
        }
    }
}

// llama_reference.cpp:72-111: per sub-block range scale and offset, 6-bit
// scales/mins relative to the block maxima, and the reference's own packing of
// sub-blocks 4..7 (low two bits in the top of bytes 0..7, high four bits in
// bytes 8..11).
void quantize_q4_K_row(const float *x, pfng_block_q4_K *y, size_t k) {
    for (size_t b = 0; b < k / PFNG_QK_K; ++b) {
        const float *v = x + b * PFNG_QK_K;
        pfng_block_q4_K &o = y[b];
        float ls[8], lm[8], maxs = 0.0f, maxm = 0.0f;
        for (int sb = 0; sb < 8; ++sb) {
            float lo = v[sb * 32], hi = lo;
            for (int j = 1; j < 32; ++j) {
                lo = std::min(lo, v[sb * 32 + j]);
                hi = std::max(hi, v[sb * 32 + j]);
            }
            ls[sb] = (hi - lo) / 15.0f;
            lm[sb] = -lo / (ls[sb] != 0.0f ? ls[sb] : 1.0f);
            maxs = std::max(maxs, ls[sb]);
            maxm = std::max(maxm, lm[sb]);
        }
        const float ds = maxs / 63.0f, dm = maxm / 63.0f;
        o.d = to_fp16(ds);
        o.dmin = to_fp16(dm);
        uint8_t s[8], m[8];
        for (int i = 0; i < 8; ++i) {
            s[i] = (uint8_t)std::min(63, (int)std::round(ls[i] / (ds != 0.0f ? ds : 1.0f)));
            m[i] = (uint8_t)std::min(63, (int)std::round(lm[i] / (dm != 0.0f ? dm : 1.0f)));
        }
        for (int i = 0; i < 4; ++i) {
            o.scales[i] = (uint8_t)(s[i] | ((s[i + 4] & 3) << 6));
            o.scales[i + 4] = (uint8_t)(m[i] | ((m[i + 4] & 3) << 6));
            o.scales[i + 8] = (uint8_t)((s[i + 4] >> 2) | ((m[i + 4] >> 2) << 4));
        }
        for (int p = 0; p < 4; ++p)
            for (int j = 0; j < 32; ++j) {
                int q[2];
                for (int h = 0; h < 2; ++h) {
                    const int sb = 2 * p + h;
                    const float t = v[sb * 32 + j] / (ls[sb] != 0.0f ? ls[sb] : 1.0f) + lm[sb];
                    q[h] = std::clamp((int)std::round(t), 0, 15);
                }
                o.qs[p * 32 + j] = (uint8_t)(q[0] | (q[1] << 4));
            }
    }
}

void fill_uniform(float *x, size_t count, std::mt19937 &g) {
    std::uniform_real_distribution<float> dist(-1.0f, 1.0f);
    for (size_t i = 0; i < count; ++i) x[i] = dist(g);
}

}  // namespace

extern "C" {

uint16_t pfng_host_fp32_to_fp16(float value) { return to_fp16(value); }
float pfng_host_fp16_to_fp32(uint16_t value) { return from_fp16(value); }

double pfng_host_checksum(const float *out, size_t count) {
    double sum = 0.0;
    for (size_t i = 0; i < count; i += 257) sum += out[i];
    return sum;
}

int pfng_host_quantize_weights(int type, const float *x, void *y, size_t rows, size_t k) {
    if (type == PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0) {
        if (k % PFNG_QK4_0) return -1;
        for (size_t r = 0; r < rows; ++r)
            quantize_q4_0_row(x + r * k, static_cast<pfng_block_q4_0 *>(y) + r * (k / PFNG_QK4_0), k);
        return 0;
    }
    if (type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K) {
        if (k % PFNG_QK_K) return -1;
        for (size_t r = 0; r < rows; ++r)
            quantize_q4_K_row(x + r * k, static_cast<pfng_block_q4_K *>(y) + r * (k / PFNG_QK_K), k);
        return 0;
    }
    return -2;
}

// benchmark.cpp:29-94
int pfng_host_create_input(int type, int variant, uint32_t seed, size_t m, size_t n, size_t k, float *activation,
                           void *weight) {
    if (variant != PFNG_INPUT_REFERENCE && variant != PFNG_INPUT_BASELINE) return -2;
    std::mt19937 g(seed);
    if (type == PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0 || type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K) {
        const size_t qk = type == PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0 ? PFNG_QK4_0 : PFNG_QK_K;
        if (k % qk) return -1;
        std::vector<float> wf;
        try {
            wf.resize(n * k);
        } catch (const std::bad_alloc &) {
            return -3;
        }
        fill_uniform(activation, m * k, g);
        fill_uniform(wf.data(), n * k, g);
        return pfng_host_quantize_weights(type, wf.data(), weight, n, k);
    }
    if (type == PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K) {
        if (k % PFNG_QK_K) return -1;
        fill_uniform(activation, m * k, g);
        const bool ref = variant == PFNG_INPUT_REFERENCE;
        std::uniform_int_distribution<unsigned> byte(0, 255);
        std::uniform_int_distribution<unsigned> grid_index(0, ref ? 31u : 255u);
        std::uniform_real_distribution<float> scale(ref ? 0.002f : 0.001f, ref ? 0.02f : 0.01f);
        auto *blocks = static_cast<pfng_block_iq2_xxs *>(weight);
        for (size_t i = 0; i < n * (k / PFNG_QK_K); ++i) {
            blocks[i].d = to_fp16(scale(g));
            auto *packed = reinterpret_cast<uint8_t *>(blocks[i].qs);
            for (size_t sb = 0; sb < PFNG_QK_K / 32; ++sb) {
                for (size_t group = 0; group < 4; ++group) packed[sb * 8 + group] = (uint8_t)grid_index(g);
                uint32_t ss = byte(g) & 0x7f;
                ss |= (byte(g) & 0x7f) << 7;
                ss |= (byte(g) & 0x7f) << 14;
                ss |= (byte(g) & 0x7f) << 21;
                ss |= (byte(g) & 0x0f) << 28;
                std::memcpy(packed + sb * 8 + 4, &ss, sizeof ss);
            }
        }
        return 0;
    }
    return -2;
}

}  // extern "C"
