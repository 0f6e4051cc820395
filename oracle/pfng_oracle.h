/*
 * TEST INFRASTRUCTURE — CPU oracle for the quantized GGML GEMM path.
 *
 * A plain-C restatement of the reference's scalar implementation
 * (bench/llama_reference/llama_reference.cpp, include/ggml.h,
 * kernels/common/iq2_xxs.h, bench/framework/benchmark.cpp input generation).
 * It exists only to check the HIP path: tests/, __graft_entry__.smoke() and
 * the cpu_baseline leg of bench.py may load it; nothing in the product does.
 *
 * Floating-point semantics follow the reference as built for x86-64 with
 * -ffp-contract=off (no FMA contraction): every expression below is evaluated
 * in fp32 in the same order as the reference source.
 */
#ifndef PFNG_ORACLE_H
#define PFNG_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "pfng_blocks.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 <-> fp32 (include/ggml.h:83-117) ---- */
float pfo_fp16_to_fp32(uint16_t h);
uint16_t pfo_fp32_to_fp16(float f);
void pfo_fp16_to_fp32_n(const uint16_t *h, float *f, size_t n);
void pfo_fp32_to_fp16_n(const float *f, uint16_t *h, size_t n);

/* ---- std::mt19937 and libstdc++ distributions (benchmark.cpp:29-32,77-79) ---- */
typedef struct {
    uint32_t state[624];
    uint32_t index;
} pfo_mt19937;

void pfo_mt_seed(pfo_mt19937 *g, uint32_t seed);
uint32_t pfo_mt_next(pfo_mt19937 *g);
float pfo_uniform_real(pfo_mt19937 *g, float a, float b);
uint32_t pfo_uniform_int(pfo_mt19937 *g, uint32_t a, uint32_t b);
/* Convenience for tests: n raw draws / n uniform_real draws from a fresh seed. */
void pfo_mt_draws(uint32_t seed, uint32_t *out, size_t n);
void pfo_uniform_real_draws(uint32_t seed, float a, float b, float *out, size_t n);

/* ---- quantizers (llama_reference.cpp:13-111) ---- */
void pfo_quantize_row_q4_0(const float *x, pfng_block_q4_0 *y, size_t count);
void pfo_quantize_row_q8_0(const float *x, pfng_block_q8_0 *y, size_t count);
void pfo_quantize_row_q8_K(const float *x, pfng_block_q8_K *y, size_t count);
void pfo_quantize_row_q4_K(const float *x, pfng_block_q4_K *y, size_t count);
/* rows x k matrices, row-major, quantized row by row */
void pfo_quantize_q8_0(const float *x, pfng_block_q8_0 *y, size_t rows, size_t k);
void pfo_quantize_q8_K(const float *x, pfng_block_q8_K *y, size_t rows, size_t k);

/* ---- dots (llama_reference.cpp:113-161) ---- */
float pfo_dot_q4_0_q8_0(const pfng_block_q4_0 *w, const pfng_block_q8_0 *a, size_t blocks);
float pfo_dot_q4_K_q8_K(const pfng_block_q4_K *w, const pfng_block_q8_K *a);
float pfo_dot_iq2_xxs_q8_K(const pfng_block_iq2_xxs *w, const pfng_block_q8_K *a);

/* IQ2_XXS sub-block decode (kernels/common/iq2_xxs.h:29-41, 256-entry grid). */
void pfo_iq2_xxs_decode_subblock(const uint8_t *packed, int8_t values[32], int *scale);
/* q4_K 6-bit scale/min unpack, the decode half of llama_reference.cpp:116-121. */
void pfo_q4_K_scales_mins(const pfng_block_q4_K *w, uint8_t scales[8], uint8_t mins[8]);

/* ---- integer block sums: the exact integer part of each dot ----
 * q4_0: out[(m*n_cols + n)*nb + b] = sum_i (q_w-8)*q_a over block b (int32, llama_reference.cpp:138-142)
 * q4_K: out2[...*2+0] = sum_j sc_j * S_j, out2[...*2+1] = sum_j m_j*(bsum_2j + bsum_2j+1)
 *       per super-block (the integer restatement of llama_reference.cpp:125-131)
 * iq2 : out[...] = sum_j (2 s_j + 1) * S_j per super-block (llama_reference.cpp:150-159) */
void pfo_isums_q4_0_q8_0(const pfng_block_q4_0 *w, const pfng_block_q8_0 *a, size_t m, size_t n, size_t k,
                         int32_t *out);
void pfo_isums_q4_K_q8_K(const pfng_block_q4_K *w, const pfng_block_q8_K *a, size_t m, size_t n, size_t k,
                         int32_t *out2);
void pfo_isums_iq2_xxs_q8_K(const pfng_block_iq2_xxs *w, const pfng_block_q8_K *a, size_t m, size_t n,
                            size_t k, int32_t *out);

/* ---- GEMM drivers (llama_reference.cpp:165-215) ----
 * compute: quantize activations, then C[m*n_cols+n] = sum over blocks, in the
 * reference's loop order. threads <= 0 uses the OpenMP default. */
int pfo_compute(int type, const float *activation, const void *weight, float *out, size_t m, size_t n, size_t k,
                int threads);
/* Same GEMM on already-quantized activations (q8_0 for type 0, q8_K otherwise). */
int pfo_matmul(int type, const void *weight, const void *act_q, float *out, size_t m, size_t n, size_t k,
               int threads);

/* ---- tolerance model ----
 * abs_terms[m*n_cols+n] = sum of |products| entering the output in exact
 * arithmetic (computed in double); the contract is |gpu - oracle| <= 1e-5 * abs_terms. */
int pfo_abs_terms(int type, const void *weight, const void *act_q, double *abs_terms, size_t m, size_t n,
                  size_t k, int threads);

/* ---- seeded input generation (benchmark.cpp:34-94) ----
 * variant 0 = the reference generator exactly.
 * variant 1 = the baseline-config generator: identical for q4_0 and q4_K; for
 *             iq2_xxs the grid index is drawn from 0..255 (not 0..31) and d from
 *             U[0.001, 0.01) (not U[0.002, 0.02)); draw order is unchanged.
 * activation: m*k floats, weight: n*(k/QK) blocks of the type's weight format. */
int pfo_create_input(int type, int variant, uint32_t seed, size_t m, size_t n, size_t k, float *activation,
                     void *weight);

/* checksum as kernels/common/adapter_common.cpp:18-23 (every 257th element). */
double pfo_checksum(const float *out, size_t count);

#ifdef __cplusplus
}
#endif

#endif /* PFNG_ORACLE_H */
