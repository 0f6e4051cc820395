// Host evaluation of llama_reference::compute, the expected output of the
// harness's verification (bench/framework/benchmark.cpp:140 calls
// llama_reference::compute for the same purpose).
//
// Activation quantizers (llama_reference.cpp:38-70) and the three scalar dots
// (:113-161) in the reference's own fp32 operation order, compiled with
// -ffp-contract=off so that every product and sum is rounded on its own; the
// M x N loops of compute_* (:165-205) are split over host threads by output
// row, which leaves every output's own summation order unchanged, so the result
// does not depend on the thread count. The iq2_xxs grid is the full 256-entry
// table (include/pfng_iq2xxs_grid.h), so weights that use every grid index
// decode as the kernels decode them.
#include <algorithm>
#include <cmath>
#include <thread>
#include <vector>

#include "pfng_blocks.h"
#include "pfng_host.h"
#include "pfng_iq2xxs_grid.h"

namespace {

// llama_reference.cpp:38-52
void act_q8_0(const float *x, pfng_block_q8_0 *y, size_t k) {
    for (size_t b = 0; b < k / PFNG_QK8_0; ++b) {
        const float *v = x + b * PFNG_QK8_0;
        float amax = 0.0f;
        for (size_t i = 0; i < PFNG_QK8_0; ++i) amax = std::max(amax, std::fabs(v[i]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[b].d = pfng_host_fp32_to_fp16(d);
        for (size_t i = 0; i < PFNG_QK8_0; ++i) y[b].qs[i] = (int8_t)std::round(v[i] * id);
    }
}

// llama_reference.cpp:54-70
void act_q8_K(const float *x, pfng_block_q8_K *y, size_t k) {
    for (size_t b = 0; b < k / PFNG_QK_K; ++b) {
        const float *v = x + b * PFNG_QK_K;
        float amax = 0.0f;
        for (size_t i = 0; i < PFNG_QK_K; ++i) amax = std::max(amax, std::fabs(v[i]));
        y[b].d = amax / 127.0f;
        const float id = y[b].d != 0.0f ? 1.0f / y[b].d : 0.0f;
        for (size_t i = 0; i < PFNG_QK_K; ++i) y[b].qs[i] = (int8_t)std::round(v[i] * id);
        for (size_t g = 0; g < PFNG_QK_K / 16; ++g) {
            int s = 0;
            for (size_t j = 0; j < 16; ++j) s += y[b].qs[g * 16 + j];
            y[b].bsums[g] = (int16_t)s;
        }
    }
}

// llama_reference.cpp:134-146: exact int32 block sum, then sum += isum * dw * da
float dot_q4_0(const pfng_block_q4_0 *w, const pfng_block_q8_0 *a, size_t blocks) {
    float sum = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        int32_t isum = 0;
        for (size_t i = 0; i < PFNG_QK4_0 / 2; ++i) {
            isum += ((int)(w[b].qs[i] & 0x0f) - 8) * a[b].qs[i];
            isum += ((int)(w[b].qs[i] >> 4) - 8) * a[b].qs[i + PFNG_QK4_0 / 2];
        }
        sum += (float)isum * pfng_host_fp16_to_fp32(w[b].d) * pfng_host_fp16_to_fp32(a[b].d);
    }
    return sum;
}

// llama_reference.cpp:113-132: fp32 accumulation per element, scaled by a.d
float dot_q4_K(const pfng_block_q4_K &w, const pfng_block_q8_K &a) {
    uint8_t sc[8], mn[8];
    for (int i = 0; i < 4; ++i) {
        sc[i] = w.scales[i] & 63;
        sc[i + 4] = (uint8_t)((w.scales[i + 8] & 15) | ((w.scales[i] >> 6) << 4));
        mn[i] = w.scales[i + 4] & 63;
        mn[i + 4] = (uint8_t)((w.scales[i + 8] >> 4) | ((w.scales[i + 4] >> 6) << 4));
    }
    const float d = pfng_host_fp16_to_fp32(w.d), dmin = pfng_host_fp16_to_fp32(w.dmin);
    float sum = 0.0f;
    for (int sb = 0; sb < 8; ++sb)
        for (int j = 0; j < 32; ++j) {
            const uint8_t byte = w.qs[(sb / 2) * 32 + j];
            const int q = (sb & 1) ? byte >> 4 : byte & 15;
            sum += (float)a.qs[sb * 32 + j] * (d * (float)sc[sb] * (float)q - dmin * (float)mn[sb]);
        }
    return a.d * sum;
}

// llama_reference.cpp:148-161 with kernels/common/iq2_xxs.h:29-41: per
// 32-element sub-block the 8 packed bytes are 4 grid indices and a
// little-endian word holding four 7-bit sign indices and a 4-bit scale s;
// sign byte = idx | parity(idx) << 7, sub-block weight 2s + 1.
float dot_iq2_xxs(const pfng_block_iq2_xxs &w, const pfng_block_q8_K &a) {
    const uint8_t *p = reinterpret_cast<const uint8_t *>(w.qs);
    int32_t sum = 0;
    for (int sb = 0; sb < PFNG_QK_K / 32; ++sb) {
        const uint8_t *g = p + sb * 8;
        const uint32_t aux = (uint32_t)g[4] | ((uint32_t)g[5] << 8) | ((uint32_t)g[6] << 16) | ((uint32_t)g[7] << 24);
        int32_t s = 0;
        for (int q = 0; q < 4; ++q) {
            const unsigned idx = (aux >> (7 * q)) & 127u;
            const unsigned signs = idx | ((unsigned)__builtin_parity(idx) << 7);
            for (int j = 0; j < 8; ++j) {
                const int v = pfng_iq2xxs_grid_byte(g[q], j);
                s += ((signs >> j) & 1 ? -v : v) * a.qs[sb * 32 + q * 8 + j];
            }
        }
        sum += (int32_t)(2 * (aux >> 28) + 1) * s;
    }
    return 0.125f * pfng_host_fp16_to_fp32(w.d) * a.d * (float)sum;
}

template <class Fn>
void for_rows(size_t rows, size_t threads, Fn fn) {
    threads = std::max<size_t>(1, std::min(threads, rows));
    if (threads == 1) {
        fn(0, rows);
        return;
    }
    std::vector<std::thread> pool;
    const size_t per = (rows + threads - 1) / threads;
    for (size_t t = 0; t < threads; ++t) {
        const size_t r0 = t * per, r1 = std::min(rows, r0 + per);
        if (r0 < r1) pool.emplace_back(fn, r0, r1);
    }
    for (auto &th : pool) th.join();
}

}  // namespace

extern "C" int pfng_host_compute(int type, const float *activation, const void *weight, float *out, size_t m,
                                 size_t n, size_t k, size_t threads) {
    if (type < 0 || type >= PFNG_QUANTIZATION_TYPE_COUNT) return -2;
    const size_t qk = type == PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0 ? PFNG_QK8_0 : PFNG_QK_K;
    if (k == 0 || k % qk) return -1;
    if (m == 0 || n == 0) return 0;
    const size_t blocks = k / qk;
    try {
        if (type == PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0) {
            std::vector<pfng_block_q8_0> a(m * blocks);
            for (size_t r = 0; r < m; ++r) act_q8_0(activation + r * k, a.data() + r * blocks, k);
            const auto *w = static_cast<const pfng_block_q4_0 *>(weight);
            for_rows(m, threads, [&](size_t r0, size_t r1) {
                for (size_t r = r0; r < r1; ++r)
                    for (size_t c = 0; c < n; ++c) out[r * n + c] = dot_q4_0(w + c * blocks, a.data() + r * blocks, blocks);
            });
            return 0;
        }
        std::vector<pfng_block_q8_K> a(m * blocks);
        for (size_t r = 0; r < m; ++r) act_q8_K(activation + r * k, a.data() + r * blocks, k);
        // compute_q4_K / compute_iq2_xxs (:178-205): out starts at 0 and each
        // super-block's dot is added in order
        for_rows(m, threads, [&](size_t r0, size_t r1) {
            for (size_t r = r0; r < r1; ++r)
                for (size_t c = 0; c < n; ++c) {
                    float acc = 0.0f;
                    for (size_t b = 0; b < blocks; ++b)
                        acc += type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K
                                   ? dot_q4_K(static_cast<const pfng_block_q4_K *>(weight)[c * blocks + b],
                                              a[r * blocks + b])
                                   : dot_iq2_xxs(static_cast<const pfng_block_iq2_xxs *>(weight)[c * blocks + b],
                                                 a[r * blocks + b]);
                    out[r * n + c] = acc;
                }
        });
        return 0;
    } catch (...) {
        return -3;
    }
}
