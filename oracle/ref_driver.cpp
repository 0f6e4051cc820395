// TEST INFRASTRUCTURE — C-ABI wrapper around the reference's own scalar code.
//
// Compiled together with /root/reference/bench/llama_reference/llama_reference.cpp
// and /root/reference/bench/framework/benchmark.cpp (unmodified, from where they
// lie) into oracle/_ref/libpfng_ref.so by oracle/Makefile. It lets the tests pin
// the C restatement in oracle/pfng_oracle.c against the reference itself.
//
// Only benchmark.cpp's create_input() is used; its run_benchmark() (which needs
// the CMake-generated build manifest) is compiled with hidden visibility and
// dropped by --gc-sections, so no generated header or stand-in is involved.
//
// Limitation kept from the reference: kernels/common/iq2_xxs.h holds a 32-entry
// grid, so ref_dot_iq2_xxs_q8_K/ref_compute are valid only for grid indices < 32
// (the reference generator's range, benchmark.cpp:78).
#include <cstring>
#include <thread>
#include <variant>
#include <vector>

#include "benchmark.h"
#include "llama_reference.h"

#define REF_API extern "C" __attribute__((visibility("default")))

using namespace pfng::bench;

namespace {

QuantizationType to_type(int type) { return static_cast<QuantizationType>(type); }

}  // namespace

REF_API float ref_fp16_to_fp32(uint16_t h) { return ggml_compute_fp16_to_fp32(h); }
REF_API uint16_t ref_fp32_to_fp16(float f) { return ggml_compute_fp32_to_fp16(f); }

REF_API void ref_quantize_row_q4_0(const float *x, void *y, size_t count) {
    llama_reference::quantize_row_q4_0(x, static_cast<block_q4_0 *>(y), count);
}
REF_API void ref_quantize_row_q8_0(const float *x, void *y, size_t count) {
    llama_reference::quantize_row_q8_0(x, static_cast<block_q8_0 *>(y), count);
}
REF_API void ref_quantize_row_q8_K(const float *x, void *y, size_t count) {
    llama_reference::quantize_row_q8_K(x, static_cast<block_q8_K *>(y), count);
}
REF_API void ref_quantize_row_q4_K(const float *x, void *y, size_t count) {
    llama_reference::quantize_row_q4_K(x, static_cast<block_q4_K *>(y), count);
}

REF_API float ref_dot_q4_0_q8_0(const void *w, const void *a, size_t blocks) {
    return llama_reference::dot_q4_0_q8_0(std::span<const block_q4_0>(static_cast<const block_q4_0 *>(w), blocks),
                                          std::span<const block_q8_0>(static_cast<const block_q8_0 *>(a), blocks));
}
REF_API float ref_dot_q4_K_q8_K(const void *w, const void *a) {
    return llama_reference::dot_q4_K_q8_K(*static_cast<const block_q4_K *>(w), *static_cast<const block_q8_K *>(a));
}
REF_API float ref_dot_iq2_xxs_q8_K(const void *w, const void *a) {
    return llama_reference::dot_iq2_xxs_q8_K(*static_cast<const block_iq2_xxs *>(w),
                                             *static_cast<const block_q8_K *>(a));
}

// bench/framework/benchmark.cpp:102-104 (seeded generator) -> caller buffers.
REF_API int ref_create_input(int type, uint64_t seed, size_t m, size_t n, size_t k, float *activation, void *weight) {
    BenchmarkRequest request;
    request.m = m;
    request.n = n;
    request.k = k;
    request.seed = seed;
    const auto owned = create_input(to_type(type), request);
    return std::visit(
        [&](const auto &input) {
            std::memcpy(activation, input.activation.data(), input.activation.size() * sizeof(float));
            std::memcpy(weight, input.weight.data(), input.weight.size() * sizeof(input.weight[0]));
            return 0;
        },
        owned);
}

// bench/llama_reference/llama_reference.cpp:213-215 on caller buffers.
REF_API int ref_compute(int type, const float *activation, const void *weight, float *out, size_t m, size_t n,
                        size_t k) {
    const size_t qk = type == 0 ? QK4_0 : QK_K;
    const size_t blocks = n * (k / qk);
    const std::span<const float> act(activation, m * k);
    BenchmarkInput input;
    switch (type) {
    case 0: input = Q4_0Q8_0Input{m, n, k, act, {static_cast<const block_q4_0 *>(weight), blocks}}; break;
    case 1: input = Q4_KQ8_KInput{m, n, k, act, {static_cast<const block_q4_K *>(weight), blocks}}; break;
    case 2: input = IQ2_XXSQ8_KInput{m, n, k, act, {static_cast<const block_iq2_xxs *>(weight), blocks}}; break;
    default: return -2;
    }
    const auto result = llama_reference::compute(to_type(type), input);
    std::memcpy(out, result.data(), result.size() * sizeof(float));
    return 0;
}

// The loops of llama_reference.cpp:164-205 (compute_q4_0 / q4_K / iq2_xxs),
// with the output columns n split over `threads` std::threads: every output
// element is the same reference dot in the same block order, so the result
// equals ref_compute's bit for bit. This is the all-core CPU baseline.
REF_API int ref_compute_threads(int type, const float *activation, const void *weight, float *out, size_t m, size_t n,
                                size_t k, int threads) {
    if (type < 0 || type > 2 || threads < 1) return -2;
    const size_t qk = type == 0 ? QK4_0 : QK_K;
    const size_t blocks = k / qk;
    std::vector<block_q8_0> a0;
    std::vector<block_q8_K> aK;
    if (type == 0) {
        a0.resize(m * blocks);
        for (size_t i = 0; i < m; ++i) llama_reference::quantize_row_q8_0(activation + i * k, a0.data() + i * blocks, k);
    } else {
        aK.resize(m * blocks);
        for (size_t i = 0; i < m; ++i) llama_reference::quantize_row_q8_K(activation + i * k, aK.data() + i * blocks, k);
    }
    auto work = [&](size_t n0, size_t n1) {
        for (size_t i = 0; i < m; ++i)
            for (size_t j = n0; j < n1; ++j) {
                if (type == 0) {
                    const auto *w = static_cast<const block_q4_0 *>(weight);
                    out[i * n + j] = llama_reference::dot_q4_0_q8_0(std::span<const block_q4_0>(w + j * blocks, blocks),
                                                                    std::span<const block_q8_0>(a0.data() + i * blocks, blocks));
                } else {
                    float s = 0.0f;
                    for (size_t b = 0; b < blocks; ++b)
                        s += type == 1 ? llama_reference::dot_q4_K_q8_K(static_cast<const block_q4_K *>(weight)[j * blocks + b],
                                                                        aK[i * blocks + b])
                                       : llama_reference::dot_iq2_xxs_q8_K(
                                             static_cast<const block_iq2_xxs *>(weight)[j * blocks + b], aK[i * blocks + b]);
                    out[i * n + j] = s;
                }
            }
    };
    std::vector<std::thread> pool;
    const size_t t = static_cast<size_t>(threads) < n ? static_cast<size_t>(threads) : (n ? n : 1);
    for (size_t p = 0; p < t; ++p) pool.emplace_back(work, n * p / t, n * (p + 1) / t);
    for (auto &th : pool) th.join();
    return 0;
}
