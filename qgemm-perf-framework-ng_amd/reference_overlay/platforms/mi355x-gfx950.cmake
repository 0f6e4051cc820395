# Platform profile of the MI355X HIP backend for the reference's CMake build
# (variables required by cmake/PlatformConfig.cmake:14-30). The kernels run on
# one AMD Instinct MI355X (gfx950); this profile builds the host side (harness,
# adapters) for the x86-64 host with the host C++ compiler (g++ or ROCm's
# clang++), through the reference's own entry point
#   PFNG_HIP_ROOT=<this repository> ./compile-and-test.sh build \
#       --platform mi355x-gfx950 --cxx "$(command -v g++)"
# or directly
#   cmake -S <reference> -B build -G Ninja -DPFNG_TARGET_PLATFORM=mi355x-gfx950 \
#         -DCMAKE_CXX_COMPILER=g++ -DPFNG_HIP_ROOT=<this repository>
# after `make -C <this repository>/qgemm-perf-framework-ng_amd` has built
# libpfng_hip.so (device code is compiled by hipcc there, not by this build).
set(PFNG_PLATFORM_ID "mi355x-gfx950")
set(PFNG_PLATFORM_DISPLAY_NAME "AMD Instinct MI355X (gfx950)")
set(PFNG_PLATFORM_ARCH "x86-64-v3")
set(PFNG_PLATFORM_TUNE "generic")
set(PFNG_PLATFORM_COMPILE_DEFINITIONS PFNG_PLATFORM_MI355X_GFX950)
# The device is found through HIP (bench/framework/platform.cpp, patched), not
# through a Device Tree; the value below only fills the manifest.
set(PFNG_PLATFORM_DEVICE_TREE_COMPATIBLES "amd,gfx950")
# Host CPUs of one GPU's share on the MI355X box; the HIP adapters use one
# host thread, the verification reference (llama_reference::compute) one too.
set(PFNG_PLATFORM_FIRST_CPU 0)
set(PFNG_PLATFORM_LAST_CPU 15)
set(PFNG_PLATFORM_MAX_THREADS 16)
set(PFNG_PLATFORM_KERNEL_COMPILE_OPTIONS -march=${PFNG_PLATFORM_ARCH} -mtune=${PFNG_PLATFORM_TUNE})
# No vector-length pinning: the host build has no RVV code.
set(PFNG_PLATFORM_FIXED_VLEN_COMPILE_OPTIONS -O2)
# Host processor and compiler of this profile (cmake/PlatformConfig.cmake
# checks them; the RISC-V profiles keep its defaults).
set(PFNG_PLATFORM_PROCESSOR_PATTERN "x86_64|AMD64")
set(PFNG_PLATFORM_COMPILER_TARGET_PATTERN "x86_64")

# Where the backend lives: this repository, with libpfng_hip.so built in
# qgemm-perf-framework-ng_amd/ and its C-ABI headers in include/.
if(NOT DEFINED PFNG_HIP_ROOT)
    set(PFNG_HIP_ROOT "" CACHE PATH "Root of the MI355X HIP backend repository")
endif()
if(NOT DEFINED PFNG_ROCM_ROOT)
    set(PFNG_ROCM_ROOT "/opt/rocm" CACHE PATH "ROCm installation (HIP runtime headers and libamdhip64)")
endif()
if(NOT PFNG_HIP_ROOT OR NOT EXISTS "${PFNG_HIP_ROOT}/include/pfng_hip.h")
    message(FATAL_ERROR "mi355x-gfx950: set -DPFNG_HIP_ROOT to the backend repository (include/pfng_hip.h)")
endif()
