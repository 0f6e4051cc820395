/*
 * pfng_hip — C-ABI of the MI355X (gfx950) quantized GGML GEMM/GEMV path.
 *
 * This is the drop-in boundary. The reference's kernel adapters reach their
 * kernels through the KernelCallbacks table (bench/framework/kernel_registry.h:92-101);
 * a HIP adapter registered under the mi355x-gfx950 platform profile calls the
 * entry points below from its callbacks:
 *   prepare()       -> device allocation + upload, pfng_hip_quantize_* for activations
 *   run()           -> pfng_hip_mul_mat_* (asynchronous), then a stream synchronize
 *   export_output() -> download of C
 *
 * Conventions (all entry points):
 *   - Pointers are DEVICE pointers. Blocks use the byte layouts of
 *     include/pfng_blocks.h (identical to the reference include/ggml.h).
 *   - Row-major: weight row n holds k/QK blocks at weight[n*(k/QK) + b], activation
 *     row m likewise, output C[m*n_cols + n] (llama_reference.cpp:170-175).
 *   - stream is a hipStream_t (NULL = the null stream). Launches are asynchronous.
 *   - Return 0 on success, a pfng_status otherwise; pfng_hip_last_error() returns a
 *     thread-local message for the last failing call. No entry point throws.
 *   - m == 0 or n == 0 is a no-op returning 0; k must be a positive multiple of the
 *     block size (32 for q4_0/q8_0, 256 for the K-quants), else PFNG_ERR_INVALID_ARGUMENT,
 *     mirroring validate_shape (kernels/common/adapter_common.h:28-43).
 */
#ifndef PFNG_HIP_H
#define PFNG_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "pfng_blocks.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    PFNG_OK = 0,
    PFNG_ERR_INVALID_ARGUMENT = 1, /* shape, null pointer, bad type or path */
    PFNG_ERR_UNSUPPORTED = 2,      /* a forced path that cannot run this shape */
    PFNG_ERR_HIP = 3,              /* HIP runtime error (message has details) */
    PFNG_ERR_DEVICE = 4            /* current device is not a gfx950 */
} pfng_status;

/* Matrix-product implementations; PFNG_PATH_AUTO picks per shape (the GEMV
 * where it applies: up to m = 16, and its MFMA tiles up to m = 64 below
 * k = 2048 and m = 128 from there, for q4_0 at k % 256 == 0 from 512, q4_K at
 * k % 1024 == 0, iq2_xxs at k % 2048 == 0; then the MFMA GEMM tiles) and
 * returns PFNG_ERR_UNSUPPORTED when neither applies (see pfng_hip_auto_path). */
typedef enum {
    PFNG_PATH_AUTO = 0,
    PFNG_PATH_GEMV = 1,  /* the decode-batch kernels. Shapes taken:
                            q4_0: m == 1 with k % 64 == 0; m = 2..8 with
                            k % 256 == 0, or k % 64 == 0 while
                            m * (k / 64) * 76 + 16 <= 163840; m = 9..16 with
                            k % 64 == 0 under that same LDS bound; m = 9..64
                            (k < 2048) or 9..128 with k % 256 == 0, k >= 512.
                            q4_K and iq2_xxs: m <= 8 with k % 256 == 0;
                            m = 9..16 while m * (k / 256) * 320 + 3072 <= 163840;
                            m = 9..64 (k < 2048) or 9..128 with k % 1024 == 0
                            (q4_K) or k % 2048 == 0 (iq2_xxs).
                            All formats: k <= 2^24 (32-bit load offsets).
                            Kernels: wavefront-per-row GEMVs for short batches;
                            16x16 int8-MFMA tiles with K split over 16 waves
                            (wave w takes the 256-element groups w, w + 16, ...,
                            one per round; below k = 4096 some waves idle), the
                            weights decoded once per wave and round and the
                            activation rows streamed in chunks of 16, from
                            m = 3..6 by format and k (iq2_xxs at k == 4096 from
                            m = 9, m = 5..8 a tile with two-half copies) */
    PFNG_PATH_MFMA = 2,  /* int8-MFMA GEMM, LDS-staged tiles: q4_0 with k % 128 == 0,
                            q4_K and iq2_xxs for every k % 256 == 0; k <= 2^24 */
    PFNG_PATH_NAIVE = 3  /* one thread per output, the reference's exact fp32 order */
} pfng_path;

/* Message of the last failing call on this host thread ("" if none). */
const char *pfng_hip_last_error(void);

/* Library version string. */
const char *pfng_hip_version(void);

/* Checks that the current HIP device is a gfx950 (MI355X). Writes the
 * gcnArchName into arch (if non-NULL) and the CU count into cus (if non-NULL).
 * Also resolves, for this device, what the other entry points look up once per
 * device (its CU count, the address of pfng_hip_compute_noalloc's scratch), so
 * that calls made under graph capture afterwards make no such query.
 * Replaces the Device-Tree platform check of bench/framework/platform.cpp:97-133. */
int pfng_hip_device_check(char *arch, size_t arch_len, int *cus);

/* ---- activation quantization ------------------------------------------ */

/* Replaces llama_reference::quantize_row_q8_0 (bench/llama_reference/llama_reference.h:12,
 * llama_reference.cpp:38-52) applied row by row to a rows x k fp32 matrix.
 * y: rows*(k/32) block_q8_0. Bytes are identical to the reference's. */
int pfng_hip_quantize_q8_0(const float *x, void *y, int64_t rows, int64_t k, void *stream);

/* Replaces llama_reference::quantize_row_q8_K (llama_reference.h:14, .cpp:54-70),
 * including the 16 int16 bsums. y: rows*(k/256) block_q8_K. Bytes identical. */
int pfng_hip_quantize_q8_K(const float *x, void *y, int64_t rows, int64_t k, void *stream);

/* ---- matrix products on quantized operands ------------------------------ */

/* C[m x n] = W(q4_0)[n x k] . A(q8_0)[m x k]^T: the loop of dot_q4_0_q8_0 over
 * every (m, n) in compute_q4_0 (llama_reference.cpp:134-146, 172-175). */
int pfng_hip_mul_mat_q4_0_q8_0(const void *weight, const void *act_q8_0, float *out, int64_t m, int64_t n,
                               int64_t k, int path, void *stream);

/* C = sum over super-blocks of dot_q4_K_q8_K (llama_reference.cpp:113-132, 186-189). */
int pfng_hip_mul_mat_q4_K_q8_K(const void *weight, const void *act_q8_K, float *out, int64_t m, int64_t n,
                               int64_t k, int path, void *stream);

/* C = sum over super-blocks of dot_iq2_xxs_q8_K (llama_reference.cpp:148-161, 200-203),
 * with the full 256-entry IQ2_XXS grid. */
int pfng_hip_mul_mat_iq2_xxs_q8_K(const void *weight, const void *act_q8_K, float *out, int64_t m, int64_t n,
                                  int64_t k, int path, void *stream);

/* The path PFNG_PATH_AUTO takes for this shape with 16-byte-aligned weights
 * and activations and a 4-byte-aligned C: PFNG_PATH_GEMV or PFNG_PATH_MFMA;
 * PFNG_PATH_AUTO for an empty product (m == 0 or n == 0); -1 (with a message
 * in pfng_hip_last_error()) when the shape is invalid or no tiled path takes
 * it, in which case PFNG_PATH_AUTO returns PFNG_ERR_UNSUPPORTED and only
 * PFNG_PATH_NAIVE runs it. The counterpart of an adapter's validate()
 * (kernels/common/adapter_common.h:28-43) for the automatic path. Host-only:
 * touches no device. */
int pfng_hip_auto_path(int type, int64_t m, int64_t n, int64_t k);

/* Type-dispatched form; type is a pfng_quantization_type. */
int pfng_hip_mul_mat(int type, const void *weight, const void *act_q, float *out, int64_t m, int64_t n, int64_t k,
                     int path, void *stream);

/* ---- weight quantizers (setup; the reference runs them on the host) ------ */

/* Replaces quantize_row_q4_0 (llama_reference.cpp:13-36) per row: x is
 * rows x k fp32 (row-major, 16-byte aligned), y receives rows * k/32
 * block_q4_0 (2-byte aligned), byte-identical to the reference. */
int pfng_hip_quantize_q4_0(const float *x, void *y, int64_t rows, int64_t k, void *stream);

/* Replaces quantize_row_q4_K (llama_reference.cpp:72-111, with its
 * non-upstream scale packing :97-101) per row; y 16-byte aligned. */
int pfng_hip_quantize_q4_K(const float *x, void *y, int64_t rows, int64_t k, void *stream);

/* ---- end to end: llama_reference::compute on the GPU -------------------- */

/* Bytes of device workspace pfng_hip_compute needs for the quantized activations. */
size_t pfng_hip_compute_workspace_size(int type, int64_t m, int64_t k);

/* Replaces llama_reference::compute (llama_reference.h:18, .cpp:165-215):
 * quantizes the fp32 activations into workspace, then runs the product.
 * workspace must hold pfng_hip_compute_workspace_size() bytes. For q4_0 with
 * m <= 2, k % 64 == 0, m * (k / 32) * 34 <= 65536 and PFNG_PATH_AUTO or
 * PFNG_PATH_GEMV the quantization is fused into the GEMV kernel (same q8_0
 * bytes, kept in LDS) and workspace is not written; from m = 3 on the separate
 * quantize launch is cheaper than quantizing again in every workgroup. */
int pfng_hip_compute(int type, const float *activation, const void *weight, float *out, int64_t m, int64_t n,
                     int64_t k, void *workspace, size_t workspace_bytes, int path, void *stream);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): pfng_hip_compute with the same arguments and results, but
 * without a workspace. The quantized activations go to a static 16 MiB device
 * array of the library (one per device, held until the process ends), so
 * m * (k/32) * 34 bytes (q4_0) or m * (k/256) * 292 bytes (q4_K, iq2_xxs) must
 * not exceed 16 MiB (q4_0 at k = 4096: m <= 3855); larger shapes return
 * PFNG_ERR_INVALID_ARGUMENT. The call itself allocates nothing. Every call on a
 * device shares that device's array: calls that overlap on one device (other
 * streams, other host threads) race and must be serialized by the caller. The
 * array's address is looked up on the first call on a device (or by
 * pfng_hip_device_check): make that call outside graph capture; later calls may
 * be captured. */
int pfng_hip_compute_noalloc(int type, const float *activation, const void *weight, float *out, int64_t m, int64_t n,
                             int64_t k, int path, void *stream);

/* ---- diagnostics ---------------------------------------------------------- */

/* Exact integer parts of every block dot, computed by the same kernel
 * configuration (operand decode, tile, K split) that PFNG_PATH_MFMA runs for
 * this shape on the current device:
 *   q4_0   : out[(m*n + n)*(k/32) + b]     = sum (q_w - 8) * q_a over block b
 *   q4_K   : out[((m*n+n)*(k/256) + b)*2]  = sum_j sc_j*S_j, [..+1] = sum_j min_j*(bsum_2j+bsum_2j+1)
 *   iq2_xxs: out[(m*n + n)*(k/256) + b]    = sum_j (2 s_j + 1) * S_j
 * Where PFNG_PATH_MFMA runs q4_K on whole-K tiles (k = 1024 or 1536), which
 * split super-blocks between K slices and join the parts only in fp32, the
 * sums come from the 64 x 64 two-slice tiles that shape would otherwise take.
 * For verification at small sizes; not a performance path. */
int pfng_hip_block_isums(int type, const void *weight, const void *act_q, int32_t *out, int64_t m, int64_t n,
                         int64_t k, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* PFNG_HIP_H */
