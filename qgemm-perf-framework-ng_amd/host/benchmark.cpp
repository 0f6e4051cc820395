// Benchmark driver of the standalone runner. One call of run_benchmark() walks
// a kernel through the phases the reference harness defines
// (bench/framework/benchmark.cpp:106-277): validate, prepare, verify against
// llama_reference::compute, warm up, calibrate the iteration count, time the
// samples. Each phase is its own function below; a phase that fails fills in
// the result's message and ends the run.
//
// Time is host wall time around the adapters' run(), which returns only after
// the device has finished, so a sample covers launches plus completion.
#include "benchmark.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <stdexcept>
#include <thread>

#include "pfng_hip.h"
#include "pfng_host.h"

namespace pfng::bench {

BenchmarkInput OwnedQ4_0Q8_0Input::view() const { return Q4_0Q8_0Input{m, n, k, activation, weight}; }
BenchmarkInput OwnedQ4_KQ8_KInput::view() const { return Q4_KQ8_KInput{m, n, k, activation, weight}; }
BenchmarkInput OwnedIQ2_XXSQ8_KInput::view() const { return IQ2_XXSQ8_KInput{m, n, k, activation, weight}; }

namespace {

// Synthetic input of one quantization pair from the product's generator
// (pfng_host_create_input, the reference's draw order).
template <class Owned, size_t kBlockElems>
Owned generate(QuantizationType type, const BenchmarkRequest &request) {
    if (request.m == 0 || request.n == 0 || request.k == 0 || request.k % kBlockElems != 0)
        throw std::runtime_error("create_input: M, N and K must be positive with K a multiple of " +
                                 std::to_string(kBlockElems));
    Owned owned;
    owned.m = request.m;
    owned.n = request.n;
    owned.k = request.k;
    owned.activation.assign(request.m * request.k, 0.0f);
    owned.weight.resize(request.n * (request.k / kBlockElems));
    const int status = pfng_host_create_input(static_cast<int>(type), request.input_variant,
                                              static_cast<uint32_t>(request.seed), request.m, request.n, request.k,
                                              owned.activation.data(), owned.weight.data());
    if (status != 0) throw std::runtime_error("pfng_host_create_input returned " + std::to_string(status));
    return owned;
}

// Raw view of the variant's operands.
struct Operands {
    size_t m = 0, n = 0, k = 0;
    const float *activation = nullptr;
    const void *weight = nullptr;
};

Operands operands(const BenchmarkInput &input) {
    return std::visit([](const auto &in) { return Operands{in.m, in.n, in.k, in.activation.data(), in.weight.data()}; },
                      input);
}

// Owns a prepared kernel state until the end of the run (destroy() is the
// adapter's only way to release it).
class PreparedState {
  public:
    PreparedState(const KernelRegistration &kernel, KernelState state) : kernel_(kernel), state_(state) {}
    PreparedState(const PreparedState &) = delete;
    PreparedState &operator=(const PreparedState &) = delete;
    ~PreparedState() {
        if (state_) kernel_.callbacks.destroy(state_);
    }
    KernelState get() const { return state_; }

  private:
    const KernelRegistration &kernel_;
    KernelState state_;
};

double seconds_for(const KernelRegistration &kernel, KernelState state, size_t iterations) {
    kernel.callbacks.reset(state);
    const auto start = std::chrono::steady_clock::now();
    kernel.callbacks.run(state, iterations);
    return std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count();
}

size_t verification_threads() {
    const unsigned hw = std::thread::hardware_concurrency();
    return std::clamp<size_t>(hw ? hw : 1, 1, 16);
}

// Pass rule of the reference harness (benchmark.cpp:144-156): an element is
// wrong when its absolute error and its error relative to max(|expected|,
// 1e-6) both exceed 1e-3. A non-finite output is wrong as well.
void compare_outputs(const std::vector<float> &got, const std::vector<float> &want, BenchmarkResult &result) {
    result.compared_elements = got.size();
    size_t first_wrong = got.size();
    for (size_t i = 0; i < got.size(); ++i) {
        const float err = std::fabs(got[i] - want[i]);
        const float rel = err / std::max(std::fabs(want[i]), 1.0e-6f);
        result.max_absolute_error = std::max(result.max_absolute_error, err);
        result.max_relative_error = std::max(result.max_relative_error, rel);
        const bool wrong = !std::isfinite(got[i]) || (err > 1.0e-3f && rel > 1.0e-3f);
        if (!wrong) continue;
        ++result.error_elements;
        if (first_wrong == got.size()) first_wrong = i;
    }
    result.error_element_ratio =
        got.empty() ? 0.0 : static_cast<double>(result.error_elements) / static_cast<double>(got.size());
    result.verified = true;
    result.verification_passed = result.error_elements == 0;
    if (!result.verification_passed) {
        char text[192];
        std::snprintf(text, sizeof text, "output %zu is %.9g where llama_reference::compute gives %.9g", first_wrong,
                      got[first_wrong], want[first_wrong]);
        result.message = text;
    }
}

// One verification run of the kernel against the host reference.
bool verify(const KernelRegistration &kernel, KernelState state, const BenchmarkRequest &request,
            const BenchmarkInput &input, BenchmarkResult &result) {
    kernel.callbacks.reset(state);
    kernel.callbacks.run(state, 1);
    std::vector<float> got(request.m * request.n);
    const ExportResult exported = kernel.callbacks.export_output(state, got);
    if (!exported.success) {
        result.message = exported.error;
        return false;
    }
    std::vector<float> want;
    expected_output(kernel.quantization, input, want);
    if (want.size() != got.size()) {
        result.message = "the host reference could not evaluate this input";
        return false;
    }
    compare_outputs(got, want, result);
    return result.verification_passed;
}

// Iterations per sample: the requested count, or as many as fill
// target_seconds judged from one timed call.
size_t iterations_per_sample(const KernelRegistration &kernel, KernelState state, const BenchmarkRequest &request) {
    if (request.iterations) return request.iterations;
    const double one_call = std::max(seconds_for(kernel, state, 1), 1.0e-7);
    return std::max<size_t>(1, static_cast<size_t>(request.target_seconds / one_call));
}

}  // namespace

OwnedBenchmarkInput create_input(QuantizationType type, const BenchmarkRequest &request) {
    switch (type) {
    case QuantizationType::WeightQ4_0ActivationQ8_0:
        return generate<OwnedQ4_0Q8_0Input, PFNG_QK4_0>(type, request);
    case QuantizationType::WeightQ4_KActivationQ8_K:
        return generate<OwnedQ4_KQ8_KInput, PFNG_QK_K>(type, request);
    case QuantizationType::WeightIQ2_XXSActivationQ8_K:
        return generate<OwnedIQ2_XXSQ8_KInput, PFNG_QK_K>(type, request);
    default: throw std::runtime_error("create_input: unknown quantization type");
    }
}

void expected_output(QuantizationType type, const BenchmarkInput &input, std::vector<float> &out) {
    const Operands op = operands(input);
    out.assign(op.m * op.n, 0.0f);
    if (pfng_host_compute(static_cast<int>(type), op.activation, op.weight, out.data(), op.m, op.n, op.k,
                          verification_threads()) != 0)
        out.clear();
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
    if (request.samples == 0) {
        result.message = "samples must be non-zero";
        return result;
    }
    const PrepareResult prepared = kernel.callbacks.prepare(request, input);
    if (!prepared.state) {
        result.message = prepared.error.empty() ? "prepare() returned no state" : prepared.error;
        return result;
    }
    const PreparedState state(kernel, prepared.state);

    if (request.verify && !verify(kernel, state.get(), request, input, result)) return result;

    kernel.callbacks.reset(state.get());
    kernel.callbacks.run(state.get(), request.warmup_iterations);
    result.iterations = iterations_per_sample(kernel, state.get(), request);

    std::vector<double> per_call;
    per_call.reserve(request.samples);
    for (size_t s = 0; s < request.samples; ++s)
        per_call.push_back(seconds_for(kernel, state.get(), result.iterations) /
                           static_cast<double>(result.iterations));
    std::sort(per_call.begin(), per_call.end());
    result.min_seconds = per_call.front();
    result.median_seconds = per_call[per_call.size() / 2];
    result.checksum = kernel.callbacks.checksum(state.get());

    const PeakPerformance peak = kernel.callbacks.peak_performance(request);
    if (!(peak.operation_count > 0.0) || !(peak.operations_per_second > 0.0) || peak.operation_name.empty()) {
        result.message = "the kernel's peak-performance model is invalid";
        return result;
    }
    result.operations_per_second = peak.operation_count / result.median_seconds;
    result.peak_operations_per_second = peak.operations_per_second;
    result.operation_name = peak.operation_name;
    result.utilization_percent = 100.0 * result.operations_per_second / peak.operations_per_second;
    return result;
}

}  // namespace pfng::bench
