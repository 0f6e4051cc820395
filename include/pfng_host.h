/* Host-side C-ABI of the MI355X backend: synthetic benchmark inputs and the
 * host weight quantizers, as the reference harness generates them.
 *
 * These are setup functions, not part of the timed path. Python callers (the
 * bench script) and the C++ harness (host/benchmark.cpp) use them so that both
 * feed the kernels the reference's own bytes for a (seed, shape) pair.
 */
#ifndef PFNG_HOST_H
#define PFNG_HOST_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Input generators. */
enum pfng_input_variant {
    /* bench/framework/benchmark.cpp:29-94: std::mt19937(seed); activations
     * m*k then weights n*k from uniform_real_distribution<float>(-1, 1),
     * weights quantized per row; iq2_xxs blocks drawn directly (d in
     * [0.002, 0.02), grid index 0..31, 5 byte draws for signs and scale). */
    PFNG_INPUT_REFERENCE = 0,
    /* As PFNG_INPUT_REFERENCE except for iq2_xxs, whose weights follow the
     * baseline's config: d in [0.001, 0.01), grid index 0..255 (the full
     * 256-entry grid), same draw order. */
    PFNG_INPUT_BASELINE = 1,
};

/* Replaces bench/framework/benchmark.h:52 `create_input(QuantizationType,
 * const BenchmarkRequest&)` (implementation benchmark.cpp:29-94) for one type:
 * writes m*k fp32 activations (row-major) to `activation` and n*(k/QK) weight
 * blocks (include/ggml.h layouts) to `weight`. Returns 0, or -1 for a k that
 * is not a multiple of the block size, -2 for an unknown type or variant,
 * -3 when out of memory. */
int pfng_host_create_input(int type, int variant, uint32_t seed, size_t m, size_t n, size_t k, float *activation,
                           void *weight);

/* Replaces bench/llama_reference/llama_reference.h quantize_row_q4_0
 * (llama_reference.cpp:13-36) for type 0 and quantize_row_q4_K
 * (llama_reference.cpp:72-111, with its non-upstream scale packing) for type
 * 1, applied to `rows` rows of k values. Returns 0, -1 (bad k) or -2 (type
 * 2 has no quantizer in the reference). */
int pfng_host_quantize_weights(int type, const float *x, void *y, size_t rows, size_t k);

/* Replaces llama_reference::compute (bench/llama_reference/llama_reference.h:18,
 * llama_reference.cpp:165-215) on the host, as the harness's verification uses
 * it (bench/framework/benchmark.cpp:140): quantizes the m x k fp32 activations
 * (quantize_row_q8_0 / q8_K) and evaluates every output with the reference's
 * scalar dot in its fp32 order (iq2_xxs with the full 256-entry grid), over
 * `threads` host threads split by output row (the result does not depend on
 * the thread count). out: m x n fp32, row-major. Returns 0, -1 (bad k), -2
 * (unknown type) or -3 (out of memory). */
int pfng_host_compute(int type, const float *activation, const void *weight, float *out, size_t m, size_t n, size_t k,
                      size_t threads);

/* ggml_compute_fp32_to_fp16 / ggml_compute_fp16_to_fp32 (include/ggml.h:83-117). */
uint16_t pfng_host_fp32_to_fp16(float value);
float pfng_host_fp16_to_fp32(uint16_t value);

/* Sum of every 257th element, as checksum_common
 * (kernels/common/adapter_common.cpp:18-23). */
double pfng_host_checksum(const float *out, size_t count);

#ifdef __cplusplus
}
#endif

#endif /* PFNG_HOST_H */
