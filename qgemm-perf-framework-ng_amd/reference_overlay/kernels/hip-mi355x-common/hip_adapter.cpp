#include "hip_adapter.h"

#include <hip/hip_runtime_api.h>
#include <linux/perf_event.h>
#include <sys/ioctl.h>
#include <sys/syscall.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <memory>
#include <string>
#include <type_traits>
#include <variant>

#include "pfng_hip.h"

namespace pfng::bench::adapters::hip_mi355x {
namespace {

constexpr double kInt8MacsPerSecond = 2.5e15;  // MI355X dense int8 MFMA: 5.0e15 ops/s

struct Format {
    size_t block_elems;
    size_t act_block_bytes;
};

Format format_of(QuantizationType type) {
    return type == QuantizationType::WeightQ4_0ActivationQ8_0 ? Format{QK8_0, sizeof(block_q8_0)}
                                                              : Format{QK_K, sizeof(block_q8_K)};
}

struct DeviceState final : CommonState {
    QuantizationType type{};
    hipStream_t stream = nullptr;
    void *weight = nullptr;
    void *act_q = nullptr;
    float *out = nullptr;
    int status = PFNG_OK;  // first failure inside run(), which has no error channel
    std::string error;

    ~DeviceState() override {
        (void)hipFree(weight);
        (void)hipFree(act_q);
        (void)hipFree(out);
        if (stream) (void)hipStreamDestroy(stream);
    }
    size_t output_bytes() const { return m() * n() * sizeof(float); }
    void note(int code, const std::string &what) {
        if (status != PFNG_OK) return;
        status = code;
        error = what;
    }
};

std::string hip_message(const char *what, hipError_t e) { return std::string(what) + ": " + hipGetErrorString(e); }

// Host operands of the variant, if it is the variant of `type`.
bool host_operands(QuantizationType type, const BenchmarkInput &input, const float *&act, const void *&weight,
                   size_t &weight_bytes) {
    return std::visit(
        [&](const auto &in) {
            using In = std::decay_t<decltype(in)>;
            constexpr QuantizationType kOwn = std::is_same_v<In, Q4_0Q8_0Input>   ? QuantizationType::WeightQ4_0ActivationQ8_0
                                              : std::is_same_v<In, Q4_KQ8_KInput> ? QuantizationType::WeightQ4_KActivationQ8_K
                                                                                  : QuantizationType::WeightIQ2_XXSActivationQ8_K;
            act = in.activation.data();
            weight = in.weight.data();
            weight_bytes = in.weight.size_bytes();
            return kOwn == type;
        },
        input);
}

// Blocks until the stream is idle, spinning in user space.
hipError_t spin_until_idle(hipStream_t stream) {
    for (;;) {
        const hipError_t e = hipStreamQuery(stream);
        if (e != hipErrorNotReady) return e;
    }
}

bool download(DeviceState &s) {
    const hipError_t e = hipMemcpy(s.output().data(), s.out, s.output_bytes(), hipMemcpyDeviceToHost);
    if (e != hipSuccess) s.note(PFNG_ERR_HIP, hip_message("output download", e));
    return e == hipSuccess;
}

}  // namespace

ValidationResult validate(QuantizationType type, const BenchmarkRequest &request) {
    const size_t qk = format_of(type).block_elems;
    ValidationResult v = qk == QK8_0 ? validate_shape<1, 1, QK8_0>(request) : validate_shape<1, 1, QK_K>(request);
    if (!v.supported) return v;
    if (pfng_hip_auto_path(static_cast<int>(type), static_cast<int64_t>(request.m), static_cast<int64_t>(request.n),
                           static_cast<int64_t>(request.k)) < 0)
        return {false, pfng_hip_last_error()};
    return v;
}

PrepareResult prepare(QuantizationType type, const BenchmarkRequest &request, const BenchmarkInput &input) {
    const float *act_host = nullptr;
    const void *weight_host = nullptr;
    size_t weight_bytes = 0;
    if (!host_operands(type, input, act_host, weight_host, weight_bytes))
        return {nullptr, "input variant does not match the kernel's quantization pair"};
    const Format f = format_of(type);
    auto s = std::make_unique<DeviceState>();
    s->type = type;
    s->m_value = request.m;
    s->n_value = request.n;
    s->k_value = request.k;
    s->blocks_k_value = request.k / f.block_elems;
    s->output_value.assign(request.m * request.n, 0.0f);

    const size_t act_bytes = request.m * request.k * sizeof(float);
    const size_t act_q_bytes = request.m * s->blocks_k() * f.act_block_bytes;
    float *act_dev = nullptr;
    hipError_t e = hipStreamCreate(&s->stream);
    if (e == hipSuccess) e = hipMalloc(&s->weight, weight_bytes);
    if (e == hipSuccess) e = hipMalloc(&s->act_q, act_q_bytes);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void **>(&s->out), s->output_bytes());
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void **>(&act_dev), act_bytes);
    if (e == hipSuccess) e = hipMemcpy(s->weight, weight_host, weight_bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(act_dev, act_host, act_bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(act_dev);
        return {nullptr, hip_message("device setup", e)};
    }
    const int rc = type == QuantizationType::WeightQ4_0ActivationQ8_0
                       ? pfng_hip_quantize_q8_0(act_dev, s->act_q, static_cast<int64_t>(request.m),
                                                static_cast<int64_t>(request.k), s->stream)
                       : pfng_hip_quantize_q8_K(act_dev, s->act_q, static_cast<int64_t>(request.m),
                                                static_cast<int64_t>(request.k), s->stream);
    e = hipStreamSynchronize(s->stream);
    (void)hipFree(act_dev);
    if (rc != PFNG_OK) return {nullptr, std::string("activation quantization: ") + pfng_hip_last_error()};
    if (e != hipSuccess) return {nullptr, hip_message("activation quantization", e)};
    return {s.release(), {}};
}

void reset(KernelState state) {
    auto &s = *static_cast<DeviceState *>(state);
    std::fill(s.output().begin(), s.output().end(), 0.0f);
    hipError_t e = hipMemsetAsync(s.out, 0, s.output_bytes(), s.stream);
    if (e == hipSuccess) e = hipStreamSynchronize(s.stream);
    if (e != hipSuccess) s.note(PFNG_ERR_HIP, hip_message("reset", e));
}

void run(KernelState state, size_t iterations) noexcept {
    auto &s = *static_cast<DeviceState *>(state);
    for (size_t i = 0; i < iterations && s.status == PFNG_OK; ++i) {
        const int rc = pfng_hip_mul_mat(static_cast<int>(s.type), s.weight, s.act_q, s.out, static_cast<int64_t>(s.m()),
                                        static_cast<int64_t>(s.n()), static_cast<int64_t>(s.k()), PFNG_PATH_AUTO,
                                        s.stream);
        if (rc != PFNG_OK) s.note(rc, pfng_hip_last_error());
    }
    const hipError_t e = spin_until_idle(s.stream);
    if (e != hipSuccess) s.note(PFNG_ERR_HIP, hip_message("stream", e));
}

ExportResult export_output(KernelState state, std::span<float> output) {
    auto &s = *static_cast<DeviceState *>(state);
    if (s.status != PFNG_OK) return {false, s.error};
    if (!download(s)) return {false, s.error};
    return export_common(state, output);
}

double checksum(KernelState state) {
    auto &s = *static_cast<DeviceState *>(state);
    if (s.status != PFNG_OK || !download(s)) return 0.0;
    return checksum_common(state);
}

void destroy(KernelState state) noexcept { destroy_common(state); }

double host_cycles_per_second() {
    static const double measured = [] {
        perf_event_attr attr{};
        attr.type = PERF_TYPE_HARDWARE;
        attr.size = sizeof(attr);
        attr.config = PERF_COUNT_HW_CPU_CYCLES;
        attr.disabled = 1;
        attr.exclude_kernel = 1;
        attr.exclude_hv = 1;
        const int fd = static_cast<int>(syscall(__NR_perf_event_open, &attr, 0, -1, -1, PERF_FLAG_FD_CLOEXEC));
        if (fd < 0) return 0.0;
        ioctl(fd, PERF_EVENT_IOC_RESET, 0);
        ioctl(fd, PERF_EVENT_IOC_ENABLE, 0);
        const auto start = std::chrono::steady_clock::now();
        double elapsed = 0.0;
        while (elapsed < 0.05) elapsed = std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count();
        ioctl(fd, PERF_EVENT_IOC_DISABLE, 0);
        uint64_t cycles = 0;
        const bool ok = read(fd, &cycles, sizeof cycles) == static_cast<ssize_t>(sizeof cycles);
        close(fd);
        return ok ? static_cast<double>(cycles) / elapsed : 0.0;
    }();
    return measured;
}

PeakPerformance peak_i8_mac(const BenchmarkRequest &request) {
    const double hz = host_cycles_per_second();
    return {static_cast<double>(request.m) * request.n * request.k, hz > 0.0 ? kInt8MacsPerSecond / hz : 0.0,
            "i8-i32 MAC"};
}

}  // namespace pfng::bench::adapters::hip_mi355x
