#include "benchmark.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <stdexcept>

#include "device_buffer.h"
#include "pfng_hip.h"
#include "pfng_host.h"

namespace pfng::bench {

BenchmarkInput OwnedQ4_0Q8_0Input::view() const { return Q4_0Q8_0Input{m, n, k, activation, weight}; }
BenchmarkInput OwnedQ4_KQ8_KInput::view() const { return Q4_KQ8_KInput{m, n, k, activation, weight}; }
BenchmarkInput OwnedIQ2_XXSQ8_KInput::view() const { return IQ2_XXSQ8_KInput{m, n, k, activation, weight}; }

namespace {

template <class Owned>
Owned make_owned(int type, size_t qk, const BenchmarkRequest &r) {
    if (!r.m || !r.n || !r.k || r.k % qk)
        throw std::runtime_error("create_input: M, N, K must be positive and K a multiple of " + std::to_string(qk));
    Owned o;
    o.m = r.m;
    o.n = r.n;
    o.k = r.k;
    o.activation.resize(r.m * r.k);
    o.weight.resize(r.n * (r.k / qk));
    const int rc = pfng_host_create_input(type, r.input_variant, (uint32_t)r.seed, r.m, r.n, r.k, o.activation.data(),
                                          o.weight.data());
    if (rc != 0) throw std::runtime_error("create_input failed with code " + std::to_string(rc));
    return o;
}

using Clock = std::chrono::steady_clock;

double seconds_of(const KernelRegistration &kernel, KernelState state, size_t iterations) {
    const auto t0 = Clock::now();
    kernel.callbacks.run(state, iterations);
    const auto t1 = Clock::now();
    return std::chrono::duration<double>(t1 - t0).count();
}

struct Operands {
    size_t m, n, k;
    const void *act;
    const void *weight;
    size_t weight_bytes;
};

Operands operands_of(const BenchmarkInput &input) {
    return std::visit(
        [](const auto &in) {
            return Operands{in.m, in.n, in.k, in.activation.data(), in.weight.data(), in.weight.size_bytes()};
        },
        input);
}

}  // namespace

OwnedBenchmarkInput create_input(QuantizationType type, const BenchmarkRequest &request) {
    switch (type) {
    case QuantizationType::WeightQ4_0ActivationQ8_0:
        return make_owned<OwnedQ4_0Q8_0Input>(PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0, PFNG_QK4_0, request);
    case QuantizationType::WeightQ4_KActivationQ8_K:
        return make_owned<OwnedQ4_KQ8_KInput>(PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K, PFNG_QK_K, request);
    case QuantizationType::WeightIQ2_XXSActivationQ8_K:
        return make_owned<OwnedIQ2_XXSQ8_KInput>(PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K, PFNG_QK_K, request);
    default: throw std::runtime_error("create_input: unknown quantization type");
    }
}

bool reference_output(QuantizationType type, const BenchmarkInput &input, std::vector<float> &out,
                      std::string &error) {
    const Operands op = operands_of(input);
    const int t = (int)type;
    const size_t ws_bytes = pfng_hip_compute_workspace_size(t, (int64_t)op.m, (int64_t)op.k);
    DeviceBuffer act, w, c, ws;
    if (!act.allocate(op.m * op.k * sizeof(float), error) || !w.allocate(op.weight_bytes, error) ||
        !c.allocate(op.m * op.n * sizeof(float), error) || !ws.allocate(ws_bytes, error))
        return false;
    if (!act.upload(op.act, op.m * op.k * sizeof(float), error) || !w.upload(op.weight, op.weight_bytes, error))
        return false;
    const int rc = pfng_hip_compute(t, static_cast<const float *>(act.get()), w.get(), static_cast<float *>(c.get()),
                                    (int64_t)op.m, (int64_t)op.n, (int64_t)op.k, ws.get(), ws_bytes,
                                    PFNG_PATH_NAIVE, nullptr);
    if (rc != PFNG_OK) {
        error = std::string("reference (naive path): ") + pfng_hip_last_error();
        return false;
    }
    if (hipDeviceSynchronize() != hipSuccess) {
        error = "reference (naive path): device synchronize failed";
        return false;
    }
    out.resize(op.m * op.n);
    return c.download(out.data(), out.size() * sizeof(float), error);
}

BenchmarkResult run_benchmark(const KernelRegistration &kernel, const BenchmarkRequest &request,
                              const BenchmarkInput &input) {
    BenchmarkResult result;
    const ValidationResult validation = kernel.callbacks.validate(request);
    if (!validation.supported) {
        result.skipped = true;
        result.message = validation.reason;
        return result;
    }
    const PrepareResult prepared = kernel.callbacks.prepare(request, input);
    if (!prepared.state) {
        result.message = prepared.error;
        return result;
    }
    struct Cleanup {
        const KernelRegistration &kernel;
        KernelState state;
        ~Cleanup() { kernel.callbacks.destroy(state); }
    } cleanup{kernel, prepared.state};

    if (request.verify) {
        kernel.callbacks.reset(prepared.state);
        kernel.callbacks.run(prepared.state, 1);
        std::vector<float> actual(request.m * request.n);
        const ExportResult exported = kernel.callbacks.export_output(prepared.state, actual);
        if (!exported.success) {
            result.message = exported.error;
            return result;
        }
        std::vector<float> expected;
        std::string error;
        if (!reference_output(kernel.quantization, input, expected, error)) {
            result.message = error;
            return result;
        }
        result.verified = true;
        result.verification_passed = true;
        result.compared_elements = actual.size();
        for (size_t i = 0; i < actual.size(); ++i) {
            const float abs_err = std::fabs(actual[i] - expected[i]);
            const float rel_err = abs_err / std::max(std::fabs(expected[i]), 1.0e-6f);
            result.max_absolute_error = std::max(result.max_absolute_error, abs_err);
            result.max_relative_error = std::max(result.max_relative_error, rel_err);
            // a NaN in either output fails as well
            if (!(abs_err <= 1.0e-3f || rel_err <= 1.0e-3f)) {
                if (result.verification_passed) {
                    char detail[160];
                    std::snprintf(detail, sizeof detail,
                                  "output differs from llama.cpp reference at index %zu: actual=%.9g expected=%.9g", i,
                                  actual[i], expected[i]);
                    result.message = detail;
                }
                result.verification_passed = false;
                ++result.error_elements;
            }
        }
        result.error_element_ratio =
            result.compared_elements ? (double)result.error_elements / (double)result.compared_elements : 0.0;
        if (!result.verification_passed) return result;
    }

    kernel.callbacks.reset(prepared.state);
    kernel.callbacks.run(prepared.state, request.warmup_iterations);
    if (request.samples == 0) {
        result.message = "samples must be non-zero";
        return result;
    }
    size_t iterations = request.iterations;
    if (!iterations) {
        // one call, then enough calls per sample to fill target_seconds
        kernel.callbacks.reset(prepared.state);
        const double one = std::max(seconds_of(kernel, prepared.state, 1), 1e-7);
        iterations = std::max<size_t>(1, (size_t)(request.target_seconds / one));
    }
    result.iterations = iterations;
    std::vector<double> per_iteration;
    for (size_t s = 0; s < request.samples; ++s) {
        kernel.callbacks.reset(prepared.state);
        per_iteration.push_back(seconds_of(kernel, prepared.state, iterations) / (double)iterations);
    }
    std::sort(per_iteration.begin(), per_iteration.end());
    result.min_seconds = per_iteration.front();
    result.median_seconds = per_iteration[per_iteration.size() / 2];
    result.checksum = kernel.callbacks.checksum(prepared.state);
    const PeakPerformance peak = kernel.callbacks.peak_performance(request);
    if (peak.operation_count <= 0.0 || peak.operations_per_second <= 0.0 || peak.operation_name.empty()) {
        result.message = "kernel returned an invalid peak-performance model";
        return result;
    }
    result.operations_per_second = peak.operation_count / result.median_seconds;
    result.peak_operations_per_second = peak.operations_per_second;
    result.operation_name = peak.operation_name;
    result.utilization_percent = result.operations_per_second / peak.operations_per_second * 100.0;
    return result;
}

}  // namespace pfng::bench
