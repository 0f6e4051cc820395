/*
 * GGML quantized block layouts shared by the MI355X kernels, the C-ABI and the
 * CPU oracle. Byte-for-byte identical to the reference's include/ggml.h so that
 * weight and activation buffers can be handed across the boundary unchanged:
 *
 *   block_q4_0    18 B  (ggml.h:125-128)   fp16 d, 16 B of nibbles, value = (nib-8)*d
 *   block_q8_0    34 B  (ggml.h:130-133)   fp16 d, 32 x int8
 *   block_q8_K   292 B  (ggml.h:135-139)   fp32 d, 256 x int8, 16 x int16 bsums
 *   block_iq2_xxs 66 B  (ggml.h:141-144)   fp16 d, 32 x uint16 (8 B per 32-element sub-block)
 *   block_q4_K   144 B  (ggml.h:149-159)   fp16 d, fp16 dmin, 12 B packed 6-bit scales/mins, 128 B nibbles
 *
 * fp16 values are carried as raw uint16_t bit patterns (ggml.h:67-69).
 * The reference's block_q4_K overlays {d, dmin} with a uint32_t; only the byte
 * layout matters here, so the struct below uses two uint16_t fields.
 */
#ifndef PFNG_BLOCKS_H
#define PFNG_BLOCKS_H

#include <stddef.h>
#include <stdint.h>

#define PFNG_QK4_0 32
#define PFNG_QK8_0 32
#define PFNG_QK_K 256
#define PFNG_K_SCALE_SIZE 12

typedef struct {
    uint16_t d;
    uint8_t qs[PFNG_QK4_0 / 2];
} pfng_block_q4_0;

typedef struct {
    uint16_t d;
    int8_t qs[PFNG_QK8_0];
} pfng_block_q8_0;

typedef struct {
    float d;
    int8_t qs[PFNG_QK_K];
    int16_t bsums[PFNG_QK_K / 16];
} pfng_block_q8_K;

typedef struct {
    uint16_t d;
    uint16_t qs[PFNG_QK_K / 8];
} pfng_block_iq2_xxs;

typedef struct {
    uint16_t d;
    uint16_t dmin;
    uint8_t scales[PFNG_K_SCALE_SIZE];
    uint8_t qs[PFNG_QK_K / 2];
} pfng_block_q4_K;

#ifdef __cplusplus
#define PFNG_STATIC_ASSERT(c, m) static_assert(c, m)
#else
#define PFNG_STATIC_ASSERT(c, m) _Static_assert(c, m)
#endif

PFNG_STATIC_ASSERT(sizeof(pfng_block_q4_0) == 18, "block_q4_0 must be 18 bytes");
PFNG_STATIC_ASSERT(sizeof(pfng_block_q8_0) == 34, "block_q8_0 must be 34 bytes");
PFNG_STATIC_ASSERT(sizeof(pfng_block_q8_K) == 292, "block_q8_K must be 292 bytes");
PFNG_STATIC_ASSERT(sizeof(pfng_block_iq2_xxs) == 66, "block_iq2_xxs must be 66 bytes");
PFNG_STATIC_ASSERT(sizeof(pfng_block_q4_K) == 144, "block_q4_K must be 144 bytes");
PFNG_STATIC_ASSERT(offsetof(pfng_block_q4_0, qs) == 2, "q4_0 qs offset");
PFNG_STATIC_ASSERT(offsetof(pfng_block_q8_0, qs) == 2, "q8_0 qs offset");
PFNG_STATIC_ASSERT(offsetof(pfng_block_q8_K, qs) == 4, "q8_K qs offset");
PFNG_STATIC_ASSERT(offsetof(pfng_block_q8_K, bsums) == 260, "q8_K bsums offset");
PFNG_STATIC_ASSERT(offsetof(pfng_block_iq2_xxs, qs) == 2, "iq2_xxs qs offset");
PFNG_STATIC_ASSERT(offsetof(pfng_block_q4_K, dmin) == 2, "q4_K dmin offset");
PFNG_STATIC_ASSERT(offsetof(pfng_block_q4_K, scales) == 4, "q4_K scales offset");
PFNG_STATIC_ASSERT(offsetof(pfng_block_q4_K, qs) == 16, "q4_K qs offset");

/* Quantization pairs, numbered as the reference's QuantizationType
 * (bench/framework/kernel_registry.h:37-42). */
enum pfng_quantization_type {
    PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0 = 0,
    PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K = 1,
    PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K = 2,
    PFNG_QUANTIZATION_TYPE_COUNT = 3
};

#endif /* PFNG_BLOCKS_H */
