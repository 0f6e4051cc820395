#include "builtin_kernels.h"

namespace pfng::bench::adapters {

void register_builtin_kernels() {
    register_q4_0_hip_mi355x();
    register_q4_K_hip_mi355x();
    register_iq2_xxs_hip_mi355x();
}

}  // namespace pfng::bench::adapters
