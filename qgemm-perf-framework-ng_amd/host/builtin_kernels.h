// Registration functions of the HIP adapters. The reference declares its
// adapters' functions in kernels/common/adapter_common.h:76-96 and generates
// register_builtin_kernels() from the pfng_declare_kernel() entries
// (cmake/Kernel.cmake:29-37); builtin_kernels.cpp is that list for this build.
#pragma once

namespace pfng::bench::adapters {

void register_q4_0_hip_mi355x();
void register_q4_K_hip_mi355x();
void register_iq2_xxs_hip_mi355x();
void register_builtin_kernels();

}  // namespace pfng::bench::adapters
