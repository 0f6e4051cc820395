// C-ABI entry points of libpfng_hip (declared in include/pfng_hip.h).
// Validates arguments on the host, picks a kernel path and launches it
// asynchronously on the caller's stream. Errors are returned as pfng_status
// codes with a thread-local message; nothing throws across the boundary.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>

#include "kernels.h"
#include "pfng_hip.h"

namespace {

thread_local char g_error[1024] = "";

int fail(int status, const char *fmt, ...) {
    va_list args;
    va_start(args, fmt);
    std::vsnprintf(g_error, sizeof g_error, fmt, args);
    va_end(args);
    return status;
}

int hip_status(hipError_t e, const char *what) {
    if (e == hipSuccess) return PFNG_OK;
    return fail(PFNG_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int64_t block_elems(int type) { return type == PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0 ? 32 : 256; }

const char *type_name(int type) {
    switch (type) {
    case PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0: return "q4_0 x q8_0";
    case PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K: return "q4_K x q8_K";
    case PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K: return "iq2_xxs x q8_K";
    default: return "unknown";
    }
}

// The shapes each tiled path takes (gemv_supported, mfma_supported; the same
// rules as include/pfng_hip.h), for the messages of declined calls.
const char *gemv_rule(int type) {
    switch (type) {
    case PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0:
        return "the q4_0 GEMV takes m == 1 at k%64==0; m = 2..16 at k%64==0 while m*(k/64)*76+16 <= 163840 "
               "(m <= 8 also at any k%256==0); m = 9..64 (k < 2048) or 9..128 at k%256==0 from k = 512";
    case PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K:
        return "the q4_K GEMV takes m <= 8; m = 9..16 while m*(k/256)*320+3072 <= 163840; m = 9..64 at k = 1024 "
               "and 9..128 at k%1024==0 from k = 2048";
    default:
        return "the iq2_xxs GEMV takes m <= 8; m = 9..16 while m*(k/256)*320+3072 <= 163840; m = 9..128 at "
               "k%2048==0";
    }
}

const char *mfma_rule(int type) {
    return type == PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0 ? "the q4_0 MFMA GEMM takes k%128==0"
                                                    : "the MFMA GEMM takes every k%256==0";
}

// Shape checks shared by every product entry point (validate_shape,
// kernels/common/adapter_common.h:28-43: K must be a multiple of the block).
int check_shape(int type, int64_t m, int64_t n, int64_t k) {
    if (type < 0 || type >= PFNG_QUANTIZATION_TYPE_COUNT) return fail(PFNG_ERR_INVALID_ARGUMENT, "unknown type %d", type);
    if (m < 0 || n < 0) return fail(PFNG_ERR_INVALID_ARGUMENT, "m and n must be non-negative (m=%lld n=%lld)",
                                    (long long)m, (long long)n);
    const int64_t qk = block_elems(type);
    if (k <= 0 || k % qk) return fail(PFNG_ERR_INVALID_ARGUMENT, "%s: k=%lld must be a positive multiple of %lld",
                                      type_name(type), (long long)k, (long long)qk);
    if (m > INT32_MAX || n > INT32_MAX || k / qk > INT32_MAX / 2)
        return fail(PFNG_ERR_INVALID_ARGUMENT, "shape too large (m=%lld n=%lld k=%lld)", (long long)m, (long long)n,
                    (long long)k);
    return PFNG_OK;
}

std::mutex g_cus_mu;
std::map<int, int> g_cus;

// Compute units of device `dev` (queried once per device).
int device_cus(int dev) {
    std::lock_guard<std::mutex> lock(g_cus_mu);
    auto it = g_cus.find(dev);
    if (it != g_cus.end()) return it->second;
    int cus = 256;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) == hipSuccess && prop.multiProcessorCount > 0) cus = prop.multiProcessorCount;
    g_cus[dev] = cus;
    return cus;
}

// Scratch of pfng_hip_compute_noalloc: the quantized activations, in a
// file-scope device array (each device that loads the library holds its own
// copy until the process ends; no allocation call is ever made for it). In host
// code `scratch` names a host-side stand-in, not the device memory: kernels get
// the address hipGetSymbolAddress returns for the current device.
constexpr size_t kNoallocScratchBytes = size_t(16) << 20;
static __device__ __align__(256) uint8_t scratch[kNoallocScratchBytes];

std::mutex g_scratch_mu;
std::map<int, void *> g_scratch_ptr;  // device -> device address of its scratch

// The current device's scratch address, looked up once per device (with that
// device current) and kept.
int noalloc_scratch(void **ptr) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(PFNG_ERR_HIP, "hipGetDevice failed");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    auto it = g_scratch_ptr.find(dev);
    if (it == g_scratch_ptr.end()) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return fail(PFNG_ERR_HIP, "compute_noalloc: hipGetSymbolAddress(scratch) on device %d: %s",
                                               dev, hipGetErrorString(e));
        it = g_scratch_ptr.emplace(dev, p).first;
    }
    *ptr = it->second;
    return PFNG_OK;
}

int launch_mfma(int type, const void *weight, const void *act_q, float *out, int64_t m, int64_t n, int64_t k,
                hipStream_t s) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(PFNG_ERR_HIP, "hipGetDevice failed");
    const pfng::MfmaPlan plan = pfng::plan_mfma(type, m, n, k, device_cus(dev));
    return hip_status(pfng::launch_mfma_mul_mat(type, weight, act_q, out, m, n, k, plan, s), "mfma launch");
}

}  // namespace

extern "C" {

const char *pfng_hip_last_error(void) { return g_error; }

const char *pfng_hip_version(void) { return "pfng_hip 0.1.0 (gfx950)"; }

int pfng_hip_device_check(char *arch, size_t arch_len, int *cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(PFNG_ERR_HIP, "hipGetDevice failed");
    hipDeviceProp_t prop;
    const hipError_t e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return hip_status(e, "hipGetDeviceProperties");
    if (arch && arch_len) {
        std::strncpy(arch, prop.gcnArchName, arch_len - 1);
        arch[arch_len - 1] = '\0';
    }
    if (cus) *cus = prop.multiProcessorCount;
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(PFNG_ERR_DEVICE, "device %d is %s, this library is built for gfx950", dev, prop.gcnArchName);
    // resolve what later calls look up once per device (the CU count of the
    // tile plans, the no-allocation scratch address) here, outside any graph
    // capture a caller may start afterwards
    device_cus(dev);
    void *scratch_ptr = nullptr;
    return noalloc_scratch(&scratch_ptr);
}

int pfng_hip_quantize_q8_0(const float *x, void *y, int64_t rows, int64_t k, void *stream) {
    if (rows < 0 || k <= 0 || k % 32) return fail(PFNG_ERR_INVALID_ARGUMENT, "quantize_q8_0: rows=%lld k=%lld (k must be a positive multiple of 32)", (long long)rows, (long long)k);
    if (rows == 0) return PFNG_OK;
    if (!x || !y) return fail(PFNG_ERR_INVALID_ARGUMENT, "quantize_q8_0: null pointer");
    if (!aligned(x, 16) || !aligned(y, 2)) return fail(PFNG_ERR_INVALID_ARGUMENT, "quantize_q8_0: x must be 16-byte and y 2-byte aligned");
    return hip_status(pfng::launch_quantize_q8_0(x, y, rows, k, static_cast<hipStream_t>(stream)), "quantize_q8_0 launch");
}

int pfng_hip_quantize_q8_K(const float *x, void *y, int64_t rows, int64_t k, void *stream) {
    if (rows < 0 || k <= 0 || k % 256) return fail(PFNG_ERR_INVALID_ARGUMENT, "quantize_q8_K: rows=%lld k=%lld (k must be a positive multiple of 256)", (long long)rows, (long long)k);
    if (rows == 0) return PFNG_OK;
    if (!x || !y) return fail(PFNG_ERR_INVALID_ARGUMENT, "quantize_q8_K: null pointer");
    if (!aligned(x, 16) || !aligned(y, 4)) return fail(PFNG_ERR_INVALID_ARGUMENT, "quantize_q8_K: x must be 16-byte and y 4-byte aligned");
    return hip_status(pfng::launch_quantize_q8_K(x, y, rows, k, static_cast<hipStream_t>(stream)), "quantize_q8_K launch");
}

int pfng_hip_quantize_q4_0(const float *x, void *y, int64_t rows, int64_t k, void *stream) {
    if (rows < 0 || k <= 0 || k % 32) return fail(PFNG_ERR_INVALID_ARGUMENT, "quantize_q4_0: rows=%lld k=%lld (k must be a positive multiple of 32)", (long long)rows, (long long)k);
    if (rows == 0) return PFNG_OK;
    if (!x || !y) return fail(PFNG_ERR_INVALID_ARGUMENT, "quantize_q4_0: null pointer");
    if (!aligned(x, 16) || !aligned(y, 2)) return fail(PFNG_ERR_INVALID_ARGUMENT, "quantize_q4_0: x must be 16-byte and y 2-byte aligned");
    return hip_status(pfng::launch_quantize_q4_0(x, y, rows, k, static_cast<hipStream_t>(stream)), "quantize_q4_0 launch");
}

int pfng_hip_quantize_q4_K(const float *x, void *y, int64_t rows, int64_t k, void *stream) {
    if (rows < 0 || k <= 0 || k % 256) return fail(PFNG_ERR_INVALID_ARGUMENT, "quantize_q4_K: rows=%lld k=%lld (k must be a positive multiple of 256)", (long long)rows, (long long)k);
    if (rows == 0) return PFNG_OK;
    if (!x || !y) return fail(PFNG_ERR_INVALID_ARGUMENT, "quantize_q4_K: null pointer");
    if (!aligned(x, 16) || !aligned(y, 16)) return fail(PFNG_ERR_INVALID_ARGUMENT, "quantize_q4_K: x and y must be 16-byte aligned");
    return hip_status(pfng::launch_quantize_q4_K(x, y, rows, k, static_cast<hipStream_t>(stream)), "quantize_q4_K launch");
}

int pfng_hip_mul_mat(int type, const void *weight, const void *act_q, float *out, int64_t m, int64_t n, int64_t k,
                     int path, void *stream) {
    int rc = check_shape(type, m, n, k);
    if (rc) return rc;
    if (m == 0 || n == 0) return PFNG_OK;
    if (!weight || !act_q || !out) return fail(PFNG_ERR_INVALID_ARGUMENT, "%s: null pointer", type_name(type));
    // Tiled paths read blocks with dword (and 16-byte) loads.
    const bool base_aligned = aligned(weight, 16) && aligned(act_q, 16) && aligned(out, 4);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const bool gemv_ok = base_aligned && pfng::gemv_supported(type, m, k);
    const bool mfma_ok = base_aligned && pfng::mfma_supported(type, m, k);
    switch (path) {
    case PFNG_PATH_AUTO:
        // measured at 4096x4096: every GEMV that applies (up to m = 128 at the
        // tiles' k) is faster than the MFMA GEMM. When neither tiled path takes the shape
        // the call is declined (as the reference's validate_shape declines,
        // kernels/common/adapter_common.h:28-43) instead of dropping to the
        // one-thread-per-output kernel, which is 10-500x slower; the caller
        // may ask for PFNG_PATH_NAIVE explicitly.
        if (gemv_ok) return hip_status(pfng::launch_gemv(type, weight, act_q, out, m, n, k, s), "gemv launch");
        if (mfma_ok) return launch_mfma(type, weight, act_q, out, m, n, k, s);
        if (!base_aligned)
            return fail(PFNG_ERR_UNSUPPORTED,
                        "%s: the tiled paths need 16-byte aligned weights and activations and a 4-byte aligned C; "
                        "PFNG_PATH_NAIVE runs every shape in the reference's fp32 order",
                        type_name(type));
        return fail(PFNG_ERR_UNSUPPORTED,
                    "%s: no tiled path takes m=%lld k=%lld (%s; %s; both k <= %lld); PFNG_PATH_NAIVE runs every "
                    "shape in the reference's fp32 order",
                    type_name(type), (long long)m, (long long)k, gemv_rule(type), mfma_rule(type),
                    (long long)pfng::kMaxTiledK);
    case PFNG_PATH_GEMV:
        if (!gemv_ok)
            return fail(PFNG_ERR_UNSUPPORTED,
                        "%s GEMV path does not take m=%lld k=%lld: %s, k <= %lld, with 16-byte aligned weights and "
                        "activations and a 4-byte aligned C",
                        type_name(type), (long long)m, (long long)k, gemv_rule(type), (long long)pfng::kMaxTiledK);
        return hip_status(pfng::launch_gemv(type, weight, act_q, out, m, n, k, s), "gemv launch");
    case PFNG_PATH_MFMA:
        if (!mfma_ok)
            return fail(PFNG_ERR_UNSUPPORTED,
                        "%s MFMA path does not take m=%lld k=%lld: %s, k <= %lld, with 16-byte aligned weights and "
                        "activations and a 4-byte aligned C",
                        type_name(type), (long long)m, (long long)k, mfma_rule(type), (long long)pfng::kMaxTiledK);
        return launch_mfma(type, weight, act_q, out, m, n, k, s);
    case PFNG_PATH_NAIVE:
        return hip_status(pfng::launch_naive_mul_mat(type, weight, act_q, out, m, n, k, s), "naive launch");
    default: return fail(PFNG_ERR_INVALID_ARGUMENT, "unknown path %d", path);
    }
}

int pfng_hip_auto_path(int type, int64_t m, int64_t n, int64_t k) {
    if (check_shape(type, m, n, k)) return -1;
    if (m == 0 || n == 0) return PFNG_PATH_AUTO;
    if (pfng::gemv_supported(type, m, k)) return PFNG_PATH_GEMV;
    if (pfng::mfma_supported(type, m, k)) return PFNG_PATH_MFMA;
    fail(PFNG_ERR_UNSUPPORTED,
         "%s: no tiled path takes m=%lld k=%lld (%s; %s; both k <= %lld); PFNG_PATH_NAIVE runs every shape in "
         "the reference's fp32 order",
         type_name(type), (long long)m, (long long)k, gemv_rule(type), mfma_rule(type), (long long)pfng::kMaxTiledK);
    return -1;
}

int pfng_hip_mul_mat_q4_0_q8_0(const void *weight, const void *act_q8_0, float *out, int64_t m, int64_t n, int64_t k,
                               int path, void *stream) {
    return pfng_hip_mul_mat(PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0, weight, act_q8_0, out, m, n, k, path, stream);
}

int pfng_hip_mul_mat_q4_K_q8_K(const void *weight, const void *act_q8_K, float *out, int64_t m, int64_t n, int64_t k,
                               int path, void *stream) {
    return pfng_hip_mul_mat(PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K, weight, act_q8_K, out, m, n, k, path, stream);
}

int pfng_hip_mul_mat_iq2_xxs_q8_K(const void *weight, const void *act_q8_K, float *out, int64_t m, int64_t n,
                                  int64_t k, int path, void *stream) {
    return pfng_hip_mul_mat(PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K, weight, act_q8_K, out, m, n, k, path, stream);
}

size_t pfng_hip_compute_workspace_size(int type, int64_t m, int64_t k) {
    if (m <= 0 || k <= 0) return 0;
    if (type == PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0) return (size_t)m * (size_t)(k / 32) * sizeof(pfng_block_q8_0);
    return (size_t)m * (size_t)(k / 256) * sizeof(pfng_block_q8_K);
}

int pfng_hip_compute(int type, const float *activation, const void *weight, float *out, int64_t m, int64_t n,
                     int64_t k, void *workspace, size_t workspace_bytes, int path, void *stream) {
    int rc = check_shape(type, m, n, k);
    if (rc) return rc;
    if (m == 0 || n == 0) return PFNG_OK;
    if (workspace_bytes < pfng_hip_compute_workspace_size(type, m, k))
        return fail(PFNG_ERR_INVALID_ARGUMENT, "compute: workspace of %zu bytes is smaller than the %zu needed",
                    workspace_bytes, pfng_hip_compute_workspace_size(type, m, k));
    // GEMV-sized problems quantize inside the product kernel (one launch, no
    // round trip of the q8 rows through HBM); the workspace is then unused
    if ((path == PFNG_PATH_AUTO || path == PFNG_PATH_GEMV) && activation && weight && out &&
        aligned(activation, 16) && aligned(weight, 16) && aligned(out, 4) && pfng::fused_gemv_supported(type, m, k))
        return hip_status(pfng::launch_fused_gemv(type, weight, activation, out, m, n, k,
                                                  static_cast<hipStream_t>(stream)),
                          "fused gemv launch");
    // decline before quantizing when the product would be declined
    if (path == PFNG_PATH_AUTO && pfng_hip_auto_path(type, m, n, k) < 0) return PFNG_ERR_UNSUPPORTED;
    rc = type == PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0 ? pfng_hip_quantize_q8_0(activation, workspace, m, k, stream)
                                                  : pfng_hip_quantize_q8_K(activation, workspace, m, k, stream);
    if (rc) return rc;
    return pfng_hip_mul_mat(type, weight, workspace, out, m, n, k, path, stream);
}

int pfng_hip_compute_noalloc(int type, const float *activation, const void *weight, float *out, int64_t m, int64_t n,
                             int64_t k, int path, void *stream) {
    int rc = check_shape(type, m, n, k);
    if (rc) return rc;
    if (m == 0 || n == 0) return PFNG_OK;
    const size_t need = pfng_hip_compute_workspace_size(type, m, k);
    if (need > kNoallocScratchBytes)
        return fail(PFNG_ERR_INVALID_ARGUMENT,
                    "compute_noalloc: the quantized activations take %zu bytes, more than the %zu-byte static "
                    "scratch (m * k/32 * 34 for q4_0, m * k/256 * 292 for the K-quants); use pfng_hip_compute "
                    "with a workspace",
                    need, kNoallocScratchBytes);
    void *scratch_ptr = nullptr;
    rc = noalloc_scratch(&scratch_ptr);
    if (rc) return rc;
    return pfng_hip_compute(type, activation, weight, out, m, n, k, scratch_ptr, kNoallocScratchBytes, path, stream);
}

int pfng_hip_block_isums(int type, const void *weight, const void *act_q, int32_t *out, int64_t m, int64_t n,
                         int64_t k, void *stream) {
    int rc = check_shape(type, m, n, k);
    if (rc) return rc;
    if (m == 0 || n == 0) return PFNG_OK;
    if (!weight || !act_q || !out) return fail(PFNG_ERR_INVALID_ARGUMENT, "block_isums: null pointer");
    if (!aligned(weight, 16) || !aligned(act_q, 16) || !aligned(out, 4) || !pfng::mfma_supported(type, m, k))
        return fail(PFNG_ERR_UNSUPPORTED, "block_isums: %s MFMA tile path not available for k=%lld", type_name(type),
                    (long long)k);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(PFNG_ERR_HIP, "hipGetDevice failed");
    const pfng::MfmaPlan plan = pfng::plan_mfma(type, m, n, k, device_cus(dev));
    return hip_status(
        pfng::launch_mfma_block_isums(type, weight, act_q, out, m, n, k, plan, static_cast<hipStream_t>(stream)),
        "block_isums launch");
}

}  // extern "C"
