// q4_0-q8_0-HIP-mi355x: dot_q4_0_q8_0 (bench/llama_reference/llama_reference.cpp:134-146) over every (m, n) on one MI355X, through the
// backend's automatic path (pfng_hip_mul_mat with PFNG_PATH_AUTO). The
// callbacks are shared by the three HIP kernel IDs (hip_adapter.h).
#include "adapter_common.h"
#include "hip_adapter.h"

namespace pfng::bench::adapters {
namespace {

constexpr QuantizationType kPair = QuantizationType::WeightQ4_0ActivationQ8_0;

ValidationResult validate(const BenchmarkRequest &request) { return hip_mi355x::validate(kPair, request); }

PrepareResult prepare(const BenchmarkRequest &request, const BenchmarkInput &input) {
    return hip_mi355x::prepare(kPair, request, input);
}

}  // namespace

void register_q4_0_hip_mi355x() {
    register_kernel({"q4_0-q8_0-HIP-mi355x",
                     "Q4_0/Q8_0 HIP gfx950 (decode GEMVs up to M=16, MFMA tile GEMVs up to M=128 "
                     "at their K, int8 MFMA GEMM above)",
                     kPair,
                     {hip_mi355x::peak_i8_mac, validate, prepare, hip_mi355x::reset, hip_mi355x::run,
                      hip_mi355x::export_output, hip_mi355x::checksum, hip_mi355x::destroy}});
}

}  // namespace pfng::bench::adapters
