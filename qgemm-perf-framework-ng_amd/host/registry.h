// Kernel registry of the MI355X harness: the operator surface of
// bench/framework/kernel_registry.h (types :20-101, functions :112-116), with
// a time-based peak in place of the per-cycle one (a GPU kernel is timed in
// seconds, not host cycles) and no host perf-event list.
#pragma once

#include <cstddef>
#include <cstdint>
#include <span>
#include <string>
#include <string_view>
#include <variant>
#include <vector>

#include "pfng_blocks.h"

namespace pfng::bench {

// kernel_registry.h:24-35
struct BenchmarkRequest {
    size_t m = 0;
    size_t n = 0;
    size_t k = 0;
    size_t warmup_iterations = 3;
    size_t samples = 10;
    size_t iterations = 0;  // 0: calibrate to target_seconds per sample
    size_t threads = 1;     // host threads (unused by the GPU kernels)
    double target_seconds = 0.05;
    uint64_t seed = 1;
    bool verify = true;
    int input_variant = 0;  // pfng_input_variant (include/pfng_host.h)
};

// kernel_registry.h:37-42 (same order: the values are the C-ABI type codes)
enum class QuantizationType {
    WeightQ4_0ActivationQ8_0 = PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0,
    WeightQ4_KActivationQ8_K = PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K,
    WeightIQ2_XXSActivationQ8_K = PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K,
    Count = PFNG_QUANTIZATION_TYPE_COUNT,
};

std::string_view quantization_name(QuantizationType type);

// kernel_registry.h:44-68: host spans, valid while the kernels of the type run
struct Q4_0Q8_0Input {
    size_t m = 0, n = 0, k = 0;
    std::span<const float> activation;
    std::span<const pfng_block_q4_0> weight;
};
struct Q4_KQ8_KInput {
    size_t m = 0, n = 0, k = 0;
    std::span<const float> activation;
    std::span<const pfng_block_q4_K> weight;
};
struct IQ2_XXSQ8_KInput {
    size_t m = 0, n = 0, k = 0;
    std::span<const float> activation;
    std::span<const pfng_block_iq2_xxs> weight;
};

using BenchmarkInput = std::variant<Q4_0Q8_0Input, Q4_KQ8_KInput, IQ2_XXSQ8_KInput>;
using KernelState = void *;

struct ValidationResult {
    bool supported = false;
    std::string reason;
};

struct PrepareResult {
    KernelState state = nullptr;
    std::string error;
};

struct ExportResult {
    bool success = false;
    std::string error;
};

// kernel_registry.h:86-90 with a time-based peak: operation_count operations
// per run at most operations_per_second.
struct PeakPerformance {
    double operation_count = 0.0;
    double operations_per_second = 0.0;
    std::string_view operation_name;
};

// kernel_registry.h:92-101. run() is the timed region and returns only after
// the device has finished the work it launched.
struct KernelCallbacks {
    PeakPerformance (*peak_performance)(const BenchmarkRequest &request);
    ValidationResult (*validate)(const BenchmarkRequest &request);
    PrepareResult (*prepare)(const BenchmarkRequest &request, const BenchmarkInput &input);
    void (*reset)(KernelState state);
    void (*run)(KernelState state, size_t iterations) noexcept;
    ExportResult (*export_output)(KernelState state, std::span<float> row_major_output);
    double (*checksum)(KernelState state);
    void (*destroy)(KernelState state) noexcept;
};

struct KernelRegistration {
    std::string_view id;
    std::string_view name;
    QuantizationType quantization;
    KernelCallbacks callbacks;
};

// kernel_registry.cpp:18-47: registration fails closed (empty id or name,
// a missing callback or a duplicate id abort the program).
void register_kernel(const KernelRegistration &registration);
std::span<const KernelRegistration> registered_kernels();
const KernelRegistration *find_kernel(std::string_view id);

}  // namespace pfng::bench
