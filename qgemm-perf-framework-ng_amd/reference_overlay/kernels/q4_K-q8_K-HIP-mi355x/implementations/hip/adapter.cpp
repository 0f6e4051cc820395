// q4_K-q8_K-HIP-mi355x: dot_q4_K_q8_K (bench/llama_reference/llama_reference.cpp:113-132) over every (m, n) on one MI355X, through the
// backend's automatic path (pfng_hip_mul_mat with PFNG_PATH_AUTO). The
// callbacks are shared by the three HIP kernel IDs (hip_adapter.h).
#include "adapter_common.h"
#include "hip_adapter.h"

namespace pfng::bench::adapters {
namespace {

constexpr QuantizationType kPair = QuantizationType::WeightQ4_KActivationQ8_K;

ValidationResult validate(const BenchmarkRequest &request) { return hip_mi355x::validate(kPair, request); }

PrepareResult prepare(const BenchmarkRequest &request, const BenchmarkInput &input) {
    return hip_mi355x::prepare(kPair, request, input);
}

}  // namespace

void register_q4_K_hip_mi355x() {
    register_kernel({"q4_K-q8_K-HIP-mi355x",
                     "Q4_K/Q8_K HIP gfx950 (decode GEMVs up to M=16, MFMA tile GEMVs up to M=128 "
                     "at their K, int8 MFMA GEMM above)",
                     kPair,
                     {hip_mi355x::peak_i8_mac, validate, prepare, hip_mi355x::reset, hip_mi355x::run,
                      hip_mi355x::export_output, hip_mi355x::checksum, hip_mi355x::destroy}});
}

}  // namespace pfng::bench::adapters
