// Command-line driver of the MI355X harness, with the options of
// bench/main.cpp (:95-101 usage, :156-205 parsing, :207-263 report):
//   pfng_bench [--build-info|--platform-info|--check-platform|--list]
//              [--kernel ID|all] --m M --n N --k K [--warmup N] [--samples N]
//              [--iterations N] [--threads N] [--no-verify]
//              [--seed S] [--input reference|baseline]
// Host perf events do not apply to GPU kernels; time per iteration is
// measured around the adapters' synchronizing run() instead of cycles.
#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <exception>
#include <string>
#include <string_view>
#include <vector>

#include "benchmark.h"
#include "builtin_kernels.h"
#include "pfng_hip.h"
#include "pfng_host.h"

namespace {

constexpr size_t kMaxThreads = 16;  // host threads are unused by the GPU kernels

bool parse_size(const char *text, size_t &value) {
    errno = 0;
    char *end = nullptr;
    const unsigned long long parsed = std::strtoull(text, &end, 10);
    if (errno || end == text || *end || !parsed || parsed > SIZE_MAX) return false;
    value = static_cast<size_t>(parsed);
    return true;
}

void usage(const char *program) {
    std::printf("Usage: %s [--build-info|--platform-info|--check-platform|--list] [--kernel ID|all] --m M --n N --k K "
                "[--warmup N] [--samples N] [--iterations N] [--threads N] [--no-verify] [--seed S] "
                "[--input reference|baseline]\n",
                program);
}

void print_build_info() {
    std::printf("platform: mi355x-gfx950\n");
    std::printf("platform display name: AMD Instinct MI355X (gfx950)\n");
    std::printf("arch: gfx950\n");
    std::printf("library: %s\n", pfng_hip_version());
    std::printf("maximum threads: %zu\n", kMaxThreads);
}

// Device 0 must be a gfx950 (the platform check of bench/framework/platform.cpp).
bool check_platform(bool print) {
    char arch[64] = {0};
    int cus = 0;
    const int rc = pfng_hip_device_check(arch, sizeof arch, &cus);
    if (print) std::printf("detected device: %s, %d CUs\n", arch[0] ? arch : "unavailable", cus);
    if (rc != PFNG_OK) {
        std::fprintf(stderr, "platform check failed: %s\n", pfng_hip_last_error());
        return false;
    }
    return true;
}

}  // namespace

int main(int argc, char **argv) {
    using namespace pfng::bench;
    adapters::register_builtin_kernels();

    BenchmarkRequest request;
    std::string_view selected = "all";
    bool list = false, build_info = false, platform_info = false, platform_check = false;
    for (int i = 1; i < argc; ++i) {
        const std::string_view a = argv[i];
        size_t seed = 0;
        if (a == "--list")
            list = true;
        else if (a == "--build-info")
            build_info = true;
        else if (a == "--platform-info")
            platform_info = true;
        else if (a == "--check-platform")
            platform_check = true;
        else if (a == "--no-verify")
            request.verify = false;
        else if (a == "--kernel" && i + 1 < argc)
            selected = argv[++i];
        else if (a == "--m" && i + 1 < argc && parse_size(argv[++i], request.m)) {
        } else if (a == "--n" && i + 1 < argc && parse_size(argv[++i], request.n)) {
        } else if (a == "--k" && i + 1 < argc && parse_size(argv[++i], request.k)) {
        } else if (a == "--warmup" && i + 1 < argc && parse_size(argv[++i], request.warmup_iterations)) {
        } else if (a == "--samples" && i + 1 < argc && parse_size(argv[++i], request.samples)) {
        } else if (a == "--iterations" && i + 1 < argc && parse_size(argv[++i], request.iterations)) {
        } else if (a == "--threads" && i + 1 < argc && parse_size(argv[++i], request.threads) &&
                   request.threads <= kMaxThreads) {
        } else if (a == "--seed" && i + 1 < argc && parse_size(argv[++i], seed)) {
            request.seed = seed;
        } else if (a == "--input" && i + 1 < argc) {
            const std::string_view v = argv[++i];
            if (v == "reference")
                request.input_variant = PFNG_INPUT_REFERENCE;
            else if (v == "baseline")
                request.input_variant = PFNG_INPUT_BASELINE;
            else {
                usage(argv[0]);
                return 2;
            }
        } else {
            usage(argv[0]);
            return 2;
        }
    }
    if (build_info) {
        print_build_info();
        return 0;
    }
    if (list) {
        for (const auto &kernel : registered_kernels()) {
            const std::string_view q = quantization_name(kernel.quantization);
            std::printf("%-26.*s %.*s [platform=mi355x-gfx950, %.*s]\n", (int)kernel.id.size(), kernel.id.data(),
                        (int)kernel.name.size(), kernel.name.data(), (int)q.size(), q.data());
        }
        return 0;
    }
    if (!check_platform(platform_info)) return 3;
    if (platform_info || platform_check) {
        std::printf("platform check: PASS\n");
        return 0;
    }
    if (!request.m || !request.n || !request.k) {
        usage(argv[0]);
        return 2;
    }
    std::vector<const KernelRegistration *> kernels;
    if (selected == "all") {
        for (const auto &kernel : registered_kernels()) kernels.push_back(&kernel);
    } else if (const auto *kernel = find_kernel(selected)) {
        kernels.push_back(kernel);
    } else {
        std::fprintf(stderr, "unknown kernel: %.*s\n", (int)selected.size(), selected.data());
        return 2;
    }

    bool failed = false;
    for (size_t t = 0; t < (size_t)QuantizationType::Count; ++t) {
        const auto type = static_cast<QuantizationType>(t);
        bool has_kernel = false;
        for (const auto *kernel : kernels) has_kernel |= kernel->quantization == type;
        if (!has_kernel) continue;
        OwnedBenchmarkInput owner;
        try {
            owner = create_input(type, request);
        } catch (const std::exception &e) {
            for (const auto *kernel : kernels) {
                if (kernel->quantization != type) continue;
                std::printf("\n[%.*s] %.*s\nstatus: SKIP (%s)\n", (int)kernel->id.size(), kernel->id.data(),
                            (int)kernel->name.size(), kernel->name.data(), e.what());
            }
            continue;
        }
        const BenchmarkInput input = std::visit([](const auto &o) { return o.view(); }, owner);
        for (const auto *kernel : kernels) {
            if (kernel->quantization != type) continue;
            const BenchmarkResult r = run_benchmark(*kernel, request, input);
            std::printf("\n[%.*s] %.*s\n", (int)kernel->id.size(), kernel->id.data(), (int)kernel->name.size(),
                        kernel->name.data());
            if (r.skipped) {
                std::printf("status: SKIP (%s)\n", r.message.c_str());
                continue;
            }
            if (r.verified)
                std::printf("error elements: %zu/%zu (%.6f%%)\n", r.error_elements, r.compared_elements,
                            r.error_element_ratio * 100.0);
            else
                std::printf("error elements: unavailable (verification disabled or not completed)\n");
            if (!r.message.empty()) {
                std::printf("status: FAIL (%s), max_abs=%.6g, max_rel=%.6g\n", r.message.c_str(), r.max_absolute_error,
                            r.max_relative_error);
                failed = true;
                continue;
            }
            std::printf("verify: %s, max_abs=%.6g, max_rel=%.6g\n", r.verified ? "PASS" : "disabled",
                        r.max_absolute_error, r.max_relative_error);
            std::printf("time: min=%.3f us median=%.3f us iterations=%zu samples=%zu\n", r.min_seconds * 1e6,
                        r.median_seconds * 1e6, r.iterations, request.samples);
            const bool bytes = r.operation_name == "HBM byte";
            const double scale = bytes ? 1e9 : 1e12;
            std::printf("performance: %.3f %s/s, %.2f%% of %.1f %s/s\n", r.operations_per_second / scale,
                        bytes ? "GB" : "T-op", r.utilization_percent, r.peak_operations_per_second / scale,
                        bytes ? "GB" : "T-op");
            std::printf("checksum: %.9g\n", r.checksum);
        }
    }
    return failed ? 1 : 0;
}
