// Kernel IDs of the MI355X backend, registered like the reference's adapters
// (kernels/*/implementations/*/adapter.cpp; callback contract
// bench/framework/kernel_registry.h:92-101). Each adapter drives the C-ABI
// launcher (include/pfng_hip.h) only:
//   prepare : upload the weight blocks and the fp32 activations, quantize the
//             activations on the device (q8_0 / q8_K, bit-exact), keep both
//             resident; the reference quantizes in prepare() as well
//             (e.g. kernels/q4_K-q8_K-RVV-upstream/implementations/rvv/adapter.cpp).
//   run     : `iterations` launches on the adapter's stream, then a stream
//             synchronize (run() is the timed region and must not return early).
//   reset   : zero the device output.   export : copy it to the host.
//   checksum: sum of every 257th output (adapter_common.cpp:18-23).
#include <cstdio>
#include <memory>
#include <string>
#include <type_traits>
#include <variant>
#include <vector>

#include "builtin_kernels.h"
#include "device_buffer.h"
#include "pfng_hip.h"
#include "pfng_host.h"
#include "registry.h"

namespace pfng::bench::adapters {

namespace {

constexpr double kInt8PeakOps = 5.0e15;   // MI355X dense int8 MFMA
constexpr double kHbmBytesPerS = 8.0e12;  // MI355X HBM3E

struct Format {
    size_t qk, weight_bytes, act_bytes;
};

Format format_of(QuantizationType t) {
    switch (t) {
    case QuantizationType::WeightQ4_0ActivationQ8_0: return {32, 18, 34};
    case QuantizationType::WeightQ4_KActivationQ8_K: return {256, 144, 292};
    default: return {256, 66, 292};
    }
}

struct HipState {
    QuantizationType type{};
    int path = PFNG_PATH_AUTO;
    size_t m = 0, n = 0, k = 0;
    hipStream_t stream = nullptr;
    DeviceBuffer weight, act_q, out;
    int status = PFNG_OK;  // first failure seen by run()
    std::string error;

    ~HipState() {
        if (stream) (void)hipStreamDestroy(stream);
    }
};

PrepareResult prepare_common(QuantizationType type, int path, const BenchmarkRequest &r, const BenchmarkInput &input) {
    auto s = std::make_unique<HipState>();
    s->type = type;
    s->path = path;
    s->m = r.m;
    s->n = r.n;
    s->k = r.k;
    const void *w_host = nullptr;
    const float *a_host = nullptr;
    size_t w_bytes = 0;
    const bool matches = std::visit(
        [&](const auto &in) {
            using In = std::decay_t<decltype(in)>;
            constexpr QuantizationType kT = std::is_same_v<In, Q4_0Q8_0Input>   ? QuantizationType::WeightQ4_0ActivationQ8_0
                                            : std::is_same_v<In, Q4_KQ8_KInput> ? QuantizationType::WeightQ4_KActivationQ8_K
                                                                                : QuantizationType::WeightIQ2_XXSActivationQ8_K;
            w_host = in.weight.data();
            a_host = in.activation.data();
            w_bytes = in.weight.size_bytes();
            return kT == type && in.m == r.m && in.n == r.n && in.k == r.k;
        },
        input);
    if (!matches) return {nullptr, "input does not match the kernel's quantization type or the request shape"};
    const Format f = format_of(type);
    std::string err;
    if (hipStreamCreate(&s->stream) != hipSuccess) return {nullptr, "hipStreamCreate failed"};
    DeviceBuffer act;
    if (!s->weight.allocate(w_bytes, err) || !s->act_q.allocate(r.m * (r.k / f.qk) * f.act_bytes, err) ||
        !s->out.allocate(r.m * r.n * sizeof(float), err) || !act.allocate(r.m * r.k * sizeof(float), err))
        return {nullptr, err};
    if (!s->weight.upload(w_host, w_bytes, err) || !act.upload(a_host, r.m * r.k * sizeof(float), err))
        return {nullptr, err};
    const int rc = type == QuantizationType::WeightQ4_0ActivationQ8_0
                       ? pfng_hip_quantize_q8_0(static_cast<const float *>(act.get()), s->act_q.get(), (int64_t)r.m,
                                                (int64_t)r.k, s->stream)
                       : pfng_hip_quantize_q8_K(static_cast<const float *>(act.get()), s->act_q.get(), (int64_t)r.m,
                                                (int64_t)r.k, s->stream);
    if (rc != PFNG_OK) return {nullptr, std::string("activation quantize: ") + pfng_hip_last_error()};
    if (hipStreamSynchronize(s->stream) != hipSuccess) return {nullptr, "activation quantize: synchronize failed"};
    return {s.release(), {}};
}

void reset(KernelState p) {
    auto &s = *static_cast<HipState *>(p);
    if (hipMemsetAsync(s.out.get(), 0, s.m * s.n * sizeof(float), s.stream) != hipSuccess ||
        hipStreamSynchronize(s.stream) != hipSuccess) {
        if (s.status == PFNG_OK) {
            s.status = PFNG_ERR_HIP;
            s.error = "reset failed";
        }
    }
}

void run(KernelState p, size_t iterations) noexcept {
    auto &s = *static_cast<HipState *>(p);
    for (size_t i = 0; i < iterations; ++i) {
        const int rc = pfng_hip_mul_mat((int)s.type, s.weight.get(), s.act_q.get(), static_cast<float *>(s.out.get()),
                                        (int64_t)s.m, (int64_t)s.n, (int64_t)s.k, s.path, s.stream);
        if (rc != PFNG_OK) {
            if (s.status == PFNG_OK) {
                s.status = rc;
                s.error = pfng_hip_last_error();
            }
            break;
        }
    }
    if (hipStreamSynchronize(s.stream) != hipSuccess && s.status == PFNG_OK) {
        s.status = PFNG_ERR_HIP;
        s.error = "stream synchronize failed";
    }
}

ExportResult export_output(KernelState p, std::span<float> out) {
    auto &s = *static_cast<HipState *>(p);
    if (s.status != PFNG_OK) return {false, s.error};
    if (out.size() != s.m * s.n) return {false, "output size mismatch"};
    std::string err;
    if (!s.out.download(out.data(), out.size_bytes(), err)) return {false, err};
    return {true, {}};
}

double checksum(KernelState p) {
    auto &s = *static_cast<HipState *>(p);
    std::vector<float> host(s.m * s.n);
    std::string err;
    if (s.status != PFNG_OK || !s.out.download(host.data(), host.size() * sizeof(float), err)) return 0.0;
    return pfng_host_checksum(host.data(), host.size());
}

void destroy(KernelState p) noexcept { delete static_cast<HipState *>(p); }

// Time-based peak: GEMV-sized problems (m <= 8) against HBM bandwidth over
// the algorithmic bytes, larger ones against the int8 MFMA rate over 2*M*N*K.
template <QuantizationType T>
PeakPerformance peak(const BenchmarkRequest &r) {
    if (r.m <= 8) {
        const Format f = format_of(T);
        const double bytes = (double)r.n * (r.k / f.qk) * f.weight_bytes + (double)r.m * (r.k / f.qk) * f.act_bytes +
                             (double)r.m * r.n * 4.0;
        return {bytes, kHbmBytesPerS, "HBM byte"};
    }
    return {2.0 * r.m * r.n * r.k, kInt8PeakOps, "int8 op"};
}

ValidationResult validate_base(QuantizationType t, const BenchmarkRequest &r) {
    if (!r.m || !r.n || !r.k) return {false, "M, N and K must be positive"};
    const size_t qk = format_of(t).qk;
    if (r.k % qk) return {false, "K must be divisible by " + std::to_string(qk)};
    return {true, {}};
}

template <QuantizationType T, int Path>
ValidationResult validate(const BenchmarkRequest &r) {
    ValidationResult v = validate_base(T, r);
    if (!v.supported) return v;
    const int auto_path = pfng_hip_auto_path((int)T, (int64_t)r.m, (int64_t)r.n, (int64_t)r.k);
    if constexpr (Path == PFNG_PATH_AUTO) {
        // the automatic path declines shapes no tiled kernel takes
        if (auto_path < 0) return {false, pfng_hip_last_error()};
    }
    if constexpr (Path == PFNG_PATH_GEMV) {
        // the automatic path prefers the GEMV wherever one applies
        if (auto_path != PFNG_PATH_GEMV)
            return {false, "no GEMV kernel takes this shape (the M and K limits of pfng_hip_auto_path)"};
    }
    if constexpr (Path == PFNG_PATH_MFMA && T == QuantizationType::WeightQ4_0ActivationQ8_0) {
        if (r.k % 128) return {false, "the q4_0 MFMA path needs K % 128 == 0"};
    }
    return v;
}

template <QuantizationType T, int Path>
PrepareResult prepare(const BenchmarkRequest &r, const BenchmarkInput &in) {
    return prepare_common(T, Path, r, in);
}

template <QuantizationType T, int Path>
void add(std::string_view id, std::string_view name) {
    register_kernel({id, name, T,
                     {peak<T>, validate<T, Path>, prepare<T, Path>, reset, run, export_output, checksum, destroy}});
}

using QT = QuantizationType;

}  // namespace

void register_q4_0_hip_mi355x() {
    add<QT::WeightQ4_0ActivationQ8_0, PFNG_PATH_AUTO>("q4_0-q8_0-HIP-mi355x",
                                                      "Q4_0/Q8_0 HIP gfx950 "
                                                      "(decode GEMVs up to M=16, MFMA tile GEMVs up to M=128 "
                                                      "at their K, int8 MFMA GEMM above)");
    add<QT::WeightQ4_0ActivationQ8_0, PFNG_PATH_GEMV>("q4_0-q8_0-HIP-gemv",
                                                      "Q4_0/Q8_0 HIP gfx950 decode GEMVs (wave-per-row and MFMA tiles)");
    add<QT::WeightQ4_0ActivationQ8_0, PFNG_PATH_MFMA>("q4_0-q8_0-HIP-mfma", "Q4_0/Q8_0 HIP gfx950 int8 MFMA GEMM");
    add<QT::WeightQ4_0ActivationQ8_0, PFNG_PATH_NAIVE>("q4_0-q8_0-HIP-naive",
                                                       "Q4_0/Q8_0 HIP thread-per-output, reference fp32 order");
}

void register_q4_K_hip_mi355x() {
    add<QT::WeightQ4_KActivationQ8_K, PFNG_PATH_AUTO>("q4_K-q8_K-HIP-mi355x",
                                                      "Q4_K/Q8_K HIP gfx950 "
                                                      "(decode GEMVs up to M=16, MFMA tile GEMVs up to M=128 "
                                                      "at their K, int8 MFMA GEMM above)");
    add<QT::WeightQ4_KActivationQ8_K, PFNG_PATH_NAIVE>("q4_K-q8_K-HIP-naive",
                                                       "Q4_K/Q8_K HIP thread-per-output, reference fp32 order");
}

void register_iq2_xxs_hip_mi355x() {
    add<QT::WeightIQ2_XXSActivationQ8_K, PFNG_PATH_AUTO>("iq2_xxs-q8_K-HIP-mi355x",
                                                      "IQ2_XXS/Q8_K HIP gfx950 "
                                                      "(decode GEMVs up to M=16, MFMA tile GEMVs up to M=128 "
                                                      "at their K, int8 MFMA GEMM above)");
    add<QT::WeightIQ2_XXSActivationQ8_K, PFNG_PATH_NAIVE>("iq2_xxs-q8_K-HIP-naive",
                                                          "IQ2_XXS/Q8_K HIP thread-per-output, reference fp32 order");
}

}  // namespace pfng::bench::adapters
