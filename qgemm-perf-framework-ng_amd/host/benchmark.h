// Benchmark driver of the standalone runner (pfng_bench): owned inputs, the
// result record and the two entry points of bench/framework/benchmark.h
// (:8-37, :46-66, :68-70), timed in seconds around the adapters' synchronizing
// run() instead of host cycle counters. The reference harness itself runs the
// same kernels through reference_overlay/ (per-host-cycle peaks).
#pragma once

#include <variant>
#include <vector>

#include "registry.h"

namespace pfng::bench {

struct OwnedQ4_0Q8_0Input {
    size_t m = 0, n = 0, k = 0;
    std::vector<float> activation;
    std::vector<pfng_block_q4_0> weight;
    BenchmarkInput view() const;
};
struct OwnedQ4_KQ8_KInput {
    size_t m = 0, n = 0, k = 0;
    std::vector<float> activation;
    std::vector<pfng_block_q4_K> weight;
    BenchmarkInput view() const;
};
struct OwnedIQ2_XXSQ8_KInput {
    size_t m = 0, n = 0, k = 0;
    std::vector<float> activation;
    std::vector<pfng_block_iq2_xxs> weight;
    BenchmarkInput view() const;
};

using OwnedBenchmarkInput = std::variant<OwnedQ4_0Q8_0Input, OwnedQ4_KQ8_KInput, OwnedIQ2_XXSQ8_KInput>;

struct BenchmarkResult {
    bool skipped = false;
    bool verified = false;
    bool verification_passed = false;
    std::string message;
    double min_seconds = 0.0;     // per iteration, best sample
    double median_seconds = 0.0;  // per iteration, median sample
    size_t iterations = 0;
    double checksum = 0.0;
    double operations_per_second = 0.0;
    double peak_operations_per_second = 0.0;
    std::string operation_name;
    double utilization_percent = 0.0;
    float max_absolute_error = 0.0f;
    float max_relative_error = 0.0f;
    size_t error_elements = 0;
    size_t compared_elements = 0;
    double error_element_ratio = 0.0;
};

// Synthetic input for request.seed, request.m/n/k and request.input_variant,
// as the reference harness makes it (benchmark.cpp:29-94). Throws
// std::runtime_error on an invalid shape.
OwnedBenchmarkInput create_input(QuantizationType type, const BenchmarkRequest &request);

// validate -> prepare -> verify -> warm-up -> calibrate -> samples, the phases
// of the reference's run_benchmark (benchmark.cpp:106-277). The expected output
// of the verification is llama_reference::compute evaluated on the host
// (pfng_host_compute); an element fails when both its absolute and its
// relative error exceed 1e-3 (benchmark.cpp:144-156) or it is not finite.
BenchmarkResult run_benchmark(const KernelRegistration &kernel, const BenchmarkRequest &request,
                              const BenchmarkInput &input);

// llama_reference::compute for one input on the host; `out` is left empty when
// the input cannot be evaluated.
void expected_output(QuantizationType type, const BenchmarkInput &input, std::vector<float> &out);

}  // namespace pfng::bench
