// Launchers of the gfx950 kernels. Host code (api.cpp) validates arguments and
// then calls these; each returns the launch status.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pfng {

// Longest rows the tiled (GEMV and MFMA) kernels take. Their loads address
// from a tile's first row with 32-bit byte offsets (tile row * row bytes):
// at k = 2^24 the largest is 127 * 65536 * 292 = 2.43e9 (q8_K, 128-row tiles)
// and 127 * 524288 * 34 = 2.26e9 (q8_0), below 2^32. Longer rows run only on
// the naive path.
constexpr int64_t kMaxTiledK = int64_t(1) << 24;

// quantize.hip
hipError_t launch_quantize_q8_0(const float *x, void *y, int64_t rows, int64_t k, hipStream_t stream);
hipError_t launch_quantize_q8_K(const float *x, void *y, int64_t rows, int64_t k, hipStream_t stream);

// quantize_weights.hip — host quantizers of the reference, on the device
hipError_t launch_quantize_q4_0(const float *x, void *y, int64_t rows, int64_t k, hipStream_t stream);
hipError_t launch_quantize_q4_K(const float *x, void *y, int64_t rows, int64_t k, hipStream_t stream);

// naive.hip — one thread per output in the reference's exact fp32 order
hipError_t launch_naive_mul_mat(int type, const void *w, const void *a, float *c, int64_t m, int64_t n, int64_t k,
                                hipStream_t stream);

// gemv.hip (q4_0) and gemv_kquant.hip (q4_K, iq2_xxs) — m <= 16, up to 64 or 128 for the MFMA tiles
bool gemv_supported(int type, int64_t m, int64_t k);
hipError_t launch_gemv(int type, const void *w, const void *a, float *c, int64_t m, int64_t n, int64_t k,
                       hipStream_t stream);
// fused activation quantization + GEMV (q4_0, m <= 8, the m q8_0 rows fit 64 KB of LDS)
bool fused_gemv_supported(int type, int64_t m, int64_t k);
hipError_t launch_fused_gemv(int type, const void *w, const float *x, float *c, int64_t m, int64_t n, int64_t k,
                             hipStream_t stream);
// fused activation quantization + GEMV for q4_K / iq2_xxs (m == 1, the q8_K row in 64 KB of LDS)
bool kquant_fused_gemv_fits(int type, int64_t m, int64_t k);
hipError_t launch_kquant_fused_gemv(int type, const void *w, const float *x, float *c, int64_t n, int64_t k,
                                    hipStream_t stream);
// q4_K / iq2_xxs GEMV rows m = 9..16 run only with the activations staged in LDS
bool kquant_gemv_staged_fits(int64_t m, int64_t k);
// m = 9..gemv_tiles_max_m(k) at q4_K k % 1024 == 0, iq2_xxs k % 2048 == 0: MFMA tiles of 16
// weight rows over chunks of 16 activation rows
bool kquant_gemv_chunked_fits(int type, int64_t m, int64_t k);
hipError_t launch_kquant_gemv(int type, const void *w, const void *a, float *c, int64_t m, int64_t n, int64_t k,
                              hipStream_t stream);

// Launch plan of the MFMA GEMMs: the tile configuration for the shape.
struct MfmaPlan {
    int config = 0;
};

// gemm_mfma.hip
bool mfma_supported(int type, int64_t m, int64_t k);
MfmaPlan plan_mfma(int type, int64_t m, int64_t n, int64_t k, int cus);
hipError_t launch_mfma_mul_mat(int type, const void *w, const void *a, float *c, int64_t m, int64_t n, int64_t k,
                               const MfmaPlan &plan, hipStream_t stream);
// the integer block sums of the configuration `plan` selects (diagnostic)
hipError_t launch_mfma_block_isums(int type, const void *w, const void *a, int32_t *out, int64_t m, int64_t n,
                                   int64_t k, const MfmaPlan &plan, hipStream_t stream);

// gemm_small.hip — q4_0 GEMMs whose 32 x 96 tiles, all of K, fit in LDS
// (k = 1024 or 1536); one workgroup per tile, K split over the waves.
// isums != nullptr writes the block sums instead of C.
bool q4_0_small_supported(int64_t k);
hipError_t launch_q4_0_small(const void *w, const void *a, float *c, int32_t *isums, int64_t m, int64_t n,
                             int64_t k, hipStream_t stream);
// q4_K against q8_K with the same 32 x 96 whole-K tiles (k = 1024 or 1536)
bool q4_K_small_supported(int64_t k);
hipError_t launch_q4_K_small(const void *w, const void *a, float *c, int64_t m, int64_t n, int64_t k,
                             hipStream_t stream);

// gemm_kquant.hip — q4_K and iq2_xxs against q8_K
MfmaPlan plan_kquant(int type, int64_t m, int64_t n, int64_t k, int cus);
hipError_t launch_kquant_mul_mat(int type, const void *w, const void *a, float *c, int64_t m, int64_t n, int64_t k,
                                 const MfmaPlan &plan, hipStream_t stream);
hipError_t launch_kquant_block_isums(int type, const void *w, const void *a, int32_t *out, int64_t m, int64_t n,
                                     int64_t k, const MfmaPlan &plan, hipStream_t stream);

}  // namespace pfng
