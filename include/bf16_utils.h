/* bf16_utils.h - bfloat16 kernels of libgpu_engine.so (gfx950 build).
 *
 * Drop-in replacement for the reference's gpu/cuda/bf16_utils.h (lines 14-58).
 * Same signatures and return convention as kernels.h: 0 on success, -1 on an
 * invalid argument or launch error. Conversions to bf16 and fp16 round to
 * nearest even.
 */
#ifndef NG_BF16_UTILS_H
#define NG_BF16_UTILS_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces bf16_utils.h:14-21 (bf16_utils.cu:95-116). output may alias input. */
int cuda_bf16_rmsnorm(void* output, const void* input, const void* weight,
                      int num_tokens, int hidden_dim, float eps);

/* Replaces bf16_utils.h:24 (bf16_utils.cu:135-147). */
int cuda_bf16_silu(void* output, const void* input, size_t num_elements);

/* Replaces bf16_utils.h:27 (bf16_utils.cu:167-180). */
int cuda_bf16_add(void* c, const void* a, const void* b, size_t num_elements);

/* Replaces bf16_utils.h:30 (bf16_utils.cu:200-213). */
int cuda_bf16_mul(void* c, const void* a, const void* b, size_t num_elements);

/* Replaces bf16_utils.h:33 (bf16_utils.cu:230-242). Exact widening. */
int cuda_bf16_to_fp32(void* output, const void* input, size_t num_elements);

/* Replaces bf16_utils.h:36 (bf16_utils.cu:255-267). */
int cuda_fp32_to_bf16(void* output, const void* input, size_t num_elements);

/* Replaces bf16_utils.h:39 (bf16_utils.cu:284-296). */
int cuda_fp16_to_bf16(void* output, const void* input, size_t num_elements);

/* Replaces bf16_utils.h:42 (bf16_utils.cu:309-321). */
int cuda_bf16_to_fp16(void* output, const void* input, size_t num_elements);

/* Replaces bf16_utils.h:45-55 (bf16_utils.cu:380-405). output may alias input. */
int cuda_bf16_rope_with_theta(void* output, const void* input, const int* positions,
                              int batch_size, int seq_len, int num_heads, int head_dim,
                              int rope_style, float rope_theta);

/* *supported = 1 when the current device computes in bf16 (every CDNA3/CDNA4
 * device does). Replaces bf16_utils.h:58 (bf16_utils.cu:411-429). */
int cuda_check_bf16_support(int* supported);

#ifdef __cplusplus
}
#endif

#endif /* NG_BF16_UTILS_H */
