/* quantize.h - int8 absmax quantization of libgpu_engine.so (gfx950 build).
 *
 * Drop-in replacement for the reference's gpu/cuda/quantize.h (lines 12-44).
 * scale = max|x| / 127 (1 when max|x| is 0); q = clamp(rint(x / scale), -127, 127)
 * with IEEE division and round-half-to-even. The reference GPU code rounds
 * half away from zero (quantize.cu:92,228,313); this library follows the
 * round-half-to-even rule of the reference's CPU path instead.
 * None of these functions synchronises the host or allocates memory: the
 * scale is produced and consumed on the device, in stream order.
 */
#ifndef NG_QUANTIZE_H
#define NG_QUANTIZE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp16 [n] -> int8 [n] + fp32 scale[1]. Replaces quantize.h:12-17
 * (quantize.cu:97-141). */
int cuda_quantize_per_tensor(void* output, void* scale, const void* input,
                             size_t num_elements);

/* int8 [n] * fp32 scale[1] -> fp16 [n]. Replaces quantize.h:20-25
 * (quantize.cu:160-182). */
int cuda_dequantize_per_tensor(void* output, const void* input, const void* scale,
                               size_t num_elements);

/* fp16 [K, N] -> int8 [K, N] + fp32 scales[N] (per column). Replaces
 * quantize.h:28-34 (quantize.cu:233-267). */
int cuda_quantize_weights(void* output, void* scales, const void* input, int K, int N);

/* fp16 [rows, cols] -> int8 [rows, cols] + fp32 scales[rows] (per row; per
 * token when rows are tokens). Replaces quantize.h:38-44 (quantize.cu:320-354). */
int cuda_quantize_weights_per_row(void* output, void* scales, const void* input,
                                  int rows, int cols);

#ifdef __cplusplus
}
#endif

#endif /* NG_QUANTIZE_H */
