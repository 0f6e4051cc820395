// Callbacks of the MI355X HIP kernel IDs for the reference harness
// (bench/framework/kernel_registry.h:86-101), over the backend's C-ABI
// (include/pfng_hip.h). One state type serves the three quantization pairs:
//   prepare : upload the weight blocks and the fp32 activations, quantize the
//             activations on the device (q8_0 / q8_K, the reference's bytes),
//             keep both resident, as the reference's adapters quantize in
//             prepare();
//   run     : `iterations` launches of PFNG_PATH_AUTO on the adapter's stream,
//             then a busy wait for the stream (run() is the timed region and
//             the harness counts user-space host cycles, so the host thread
//             spins instead of sleeping in the driver);
//   reset   : zero the device output;  export : download it;
//   checksum: download, then checksum_common (every 257th output).
#ifndef PFNG_HIP_MI355X_ADAPTER_H
#define PFNG_HIP_MI355X_ADAPTER_H

#include "adapter_common.h"

namespace pfng::bench::adapters::hip_mi355x {

// validate_shape<1, 1, QK>, then the backend's own shape query: the automatic
// path declines shapes no tiled kernel takes (pfng_hip_auto_path).
ValidationResult validate(QuantizationType type, const BenchmarkRequest &request);
PrepareResult prepare(QuantizationType type, const BenchmarkRequest &request, const BenchmarkInput &input);
void reset(KernelState state);
void run(KernelState state, size_t iterations) noexcept;
ExportResult export_output(KernelState state, std::span<float> output);
double checksum(KernelState state);
void destroy(KernelState state) noexcept;

// M*N*K int8 MACs per run against the MI355X dense int8 MFMA rate (5.0e15
// ops/s = 2.5e15 MAC/s), expressed per cycle of the host core that times
// run(): MAC/s divided by that core's measured user-space cycles per second.
PeakPerformance peak_i8_mac(const BenchmarkRequest &request);

// User-space cycles per second of the calling host thread, from the same
// perf_event cycles counter the harness reads (measured once over a 50 ms
// spin); 0 when the counter cannot be opened.
double host_cycles_per_second();

}  // namespace pfng::bench::adapters::hip_mi355x

#endif
