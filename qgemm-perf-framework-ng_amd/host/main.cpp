// pfng_bench: standalone command-line runner of the HIP kernel IDs. It takes
// the reference's option names (bench/main.cpp:95-101) and prints its report
// lines (bench/main.cpp:236-263), so scripts written for pfng-bench read it;
// timing is wall time around the adapters' synchronizing run() (per-second
// figures instead of per-host-cycle ones).
//
//   pfng_bench [--build-info|--platform-info|--check-platform|--list]
//              [--kernel ID|all] --m M --n N --k K [--warmup N] [--samples N]
//              [--iterations N] [--threads N] [--no-verify]
//              [--seed S] [--input reference|baseline]
#include <charconv>
#include <cstdio>
#include <exception>
#include <optional>
#include <string>
#include <string_view>
#include <vector>

#include "benchmark.h"
#include "builtin_kernels.h"
#include "pfng_hip.h"
#include "pfng_host.h"

namespace {

using pfng::bench::BenchmarkRequest;

constexpr size_t kHostThreadLimit = 16;  // the GPU box's CPU share

enum class Action { Run, List, BuildInfo, PlatformInfo, CheckPlatform };

struct CommandLine {
    Action action = Action::Run;
    std::string kernel = "all";
    BenchmarkRequest request;
};

// Options that take a positive integer, and where it goes.
struct CountOption {
    std::string_view flag;
    size_t BenchmarkRequest::*field;
    size_t limit;
};
constexpr CountOption kCountOptions[] = {
    {"--m", &BenchmarkRequest::m, SIZE_MAX},
    {"--n", &BenchmarkRequest::n, SIZE_MAX},
    {"--k", &BenchmarkRequest::k, SIZE_MAX},
    {"--warmup", &BenchmarkRequest::warmup_iterations, SIZE_MAX},
    {"--samples", &BenchmarkRequest::samples, SIZE_MAX},
    {"--iterations", &BenchmarkRequest::iterations, SIZE_MAX},
    {"--threads", &BenchmarkRequest::threads, kHostThreadLimit},
};

// Options that only select what the program does.
struct ActionOption {
    std::string_view flag;
    Action action;
};
constexpr ActionOption kActionOptions[] = {
    {"--list", Action::List},
    {"--build-info", Action::BuildInfo},
    {"--platform-info", Action::PlatformInfo},
    {"--check-platform", Action::CheckPlatform},
};

// A whole-string positive decimal count.
std::optional<uint64_t> positive_count(std::string_view text) {
    uint64_t value = 0;
    const auto [end, ec] = std::from_chars(text.data(), text.data() + text.size(), value);
    if (ec != std::errc() || end != text.data() + text.size() || value == 0) return std::nullopt;
    return value;
}

// Fills `cl` from argv; false on anything it does not understand.
bool read_command_line(int argc, char **argv, CommandLine &cl) {
    for (int i = 1; i < argc; ++i) {
        const std::string_view flag = argv[i];
        const char *operand = i + 1 < argc ? argv[i + 1] : nullptr;
        bool known = false;
        for (const ActionOption &o : kActionOptions)
            if (flag == o.flag) {
                cl.action = o.action;
                known = true;
            }
        if (known) continue;
        if (flag == "--no-verify") {
            cl.request.verify = false;
            continue;
        }
        if (!operand) return false;  // every remaining option takes a value
        ++i;
        if (flag == "--kernel") {
            cl.kernel = operand;
            continue;
        }
        if (flag == "--input") {
            const std::string_view v = operand;
            if (v != "reference" && v != "baseline") return false;
            cl.request.input_variant = v == "reference" ? PFNG_INPUT_REFERENCE : PFNG_INPUT_BASELINE;
            continue;
        }
        const std::optional<uint64_t> count = positive_count(operand);
        if (!count) return false;
        if (flag == "--seed") {
            cl.request.seed = *count;
            continue;
        }
        for (const CountOption &o : kCountOptions)
            if (flag == o.flag) {
                if (*count > o.limit) return false;
                cl.request.*o.field = static_cast<size_t>(*count);
                known = true;
            }
        if (!known) return false;
    }
    return true;
}

void print_usage(const char *program) {
    std::printf("Usage: %s [--build-info|--platform-info|--check-platform|--list] [--kernel ID|all] --m M --n N --k K "
                "[--warmup N] [--samples N] [--iterations N] [--threads N] [--no-verify] [--seed S] "
                "[--input reference|baseline]\n",
                program);
}

void print_build_info() {
    std::printf("platform: mi355x-gfx950\n"
                "platform display name: AMD Instinct MI355X (gfx950)\n"
                "arch: gfx950\n"
                "library: %s\n"
                "maximum threads: %zu\n",
                pfng_hip_version(), kHostThreadLimit);
}

// The runtime platform check: device 0 must be a gfx950.
bool device_is_gfx950(bool verbose) {
    char arch[64] = "";
    int cus = 0;
    const int status = pfng_hip_device_check(arch, sizeof arch, &cus);
    if (verbose) std::printf("detected device: %s, %d CUs\n", arch[0] ? arch : "unavailable", cus);
    if (status != PFNG_OK) std::fprintf(stderr, "platform check failed: %s\n", pfng_hip_last_error());
    return status == PFNG_OK;
}

void print_catalogue() {
    for (const auto &k : pfng::bench::registered_kernels()) {
        const std::string_view q = pfng::bench::quantization_name(k.quantization);
        std::printf("%-26.*s %.*s [platform=mi355x-gfx950, %.*s]\n", static_cast<int>(k.id.size()), k.id.data(),
                    static_cast<int>(k.name.size()), k.name.data(), static_cast<int>(q.size()), q.data());
    }
}

// The report of one kernel, in the reference's line format. Returns false
// when the kernel failed.
bool report(const pfng::bench::KernelRegistration &k, const pfng::bench::BenchmarkResult &r, size_t samples) {
    std::printf("\n[%.*s] %.*s\n", static_cast<int>(k.id.size()), k.id.data(), static_cast<int>(k.name.size()),
                k.name.data());
    if (r.skipped) {
        std::printf("status: SKIP (%s)\n", r.message.c_str());
        return true;
    }
    if (r.verified)
        std::printf("error elements: %zu/%zu (%.6f%%)\n", r.error_elements, r.compared_elements,
                    100.0 * r.error_element_ratio);
    else
        std::printf("error elements: unavailable (verification disabled or not completed)\n");
    if (!r.message.empty()) {
        std::printf("status: FAIL (%s), max_abs=%.6g, max_rel=%.6g\n", r.message.c_str(), r.max_absolute_error,
                    r.max_relative_error);
        return false;
    }
    std::printf("verify: %s, max_abs=%.6g, max_rel=%.6g\n", r.verified ? "PASS" : "disabled", r.max_absolute_error,
                r.max_relative_error);
    std::printf("time: min=%.3f us median=%.3f us iterations=%zu samples=%zu\n", 1e6 * r.min_seconds,
                1e6 * r.median_seconds, r.iterations, samples);
    const bool bytes = r.operation_name == "HBM byte";
    const double unit = bytes ? 1e9 : 1e12;
    const char *unit_name = bytes ? "GB" : "T-op";
    std::printf("performance: %.3f %s/s, %.2f%% of %.1f %s/s\n", r.operations_per_second / unit, unit_name,
                r.utilization_percent, r.peak_operations_per_second / unit, unit_name);
    std::printf("checksum: %.9g\n", r.checksum);
    return true;
}

// Runs every selected kernel, one input per quantization pair.
bool run_selected(const std::vector<const pfng::bench::KernelRegistration *> &selected, const BenchmarkRequest &req) {
    using pfng::bench::QuantizationType;
    bool all_passed = true;
    for (size_t t = 0; t < static_cast<size_t>(QuantizationType::Count); ++t) {
        const auto type = static_cast<QuantizationType>(t);
        std::vector<const pfng::bench::KernelRegistration *> of_type;
        for (const auto *k : selected)
            if (k->quantization == type) of_type.push_back(k);
        if (of_type.empty()) continue;
        pfng::bench::OwnedBenchmarkInput owner;
        try {
            owner = pfng::bench::create_input(type, req);
        } catch (const std::exception &e) {
            for (const auto *k : of_type)
                std::printf("\n[%.*s] %.*s\nstatus: SKIP (%s)\n", static_cast<int>(k->id.size()), k->id.data(),
                            static_cast<int>(k->name.size()), k->name.data(), e.what());
            continue;
        }
        const pfng::bench::BenchmarkInput input = std::visit([](const auto &o) { return o.view(); }, owner);
        for (const auto *k : of_type) all_passed &= report(*k, pfng::bench::run_benchmark(*k, req, input), req.samples);
    }
    return all_passed;
}

}  // namespace

int main(int argc, char **argv) {
    pfng::bench::adapters::register_builtin_kernels();
    CommandLine cl;
    if (!read_command_line(argc, argv, cl)) {
        print_usage(argv[0]);
        return 2;
    }
    switch (cl.action) {
    case Action::BuildInfo: print_build_info(); return 0;
    case Action::List: print_catalogue(); return 0;
    case Action::PlatformInfo:
    case Action::CheckPlatform:
        if (!device_is_gfx950(cl.action == Action::PlatformInfo)) return 3;
        std::printf("platform check: PASS\n");
        return 0;
    case Action::Run: break;
    }
    if (!device_is_gfx950(false)) return 3;
    if (!cl.request.m || !cl.request.n || !cl.request.k) {
        print_usage(argv[0]);
        return 2;
    }
    std::vector<const pfng::bench::KernelRegistration *> selected;
    if (cl.kernel == "all") {
        for (const auto &k : pfng::bench::registered_kernels()) selected.push_back(&k);
    } else if (const auto *k = pfng::bench::find_kernel(cl.kernel)) {
        selected.push_back(k);
    } else {
        std::fprintf(stderr, "unknown kernel: %s\n", cl.kernel.c_str());
        return 2;
    }
    return run_selected(selected, cl.request) ? 0 : 1;
}
