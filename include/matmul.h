/* matmul.h - fp16 GEMM and int8-weight GEMM of libgpu_engine.so (gfx950 build).
 *
 * Drop-in replacement for the two GEMM entry points of the reference's
 * gpu/cuda/matmul.h (lines 16-38) that the INT8 layer path calls
 * (gpu/engine/layer.cu:487-501,551,575). All matrices are row-major.
 *
 * cuda_gemm_int8 computes C[M,N] = A[M,K] @ (B * scale)^T when transpose_b
 * (B int8 [N,K], scale[n] per row of B, the engine's layout), or
 * A @ (B * scale) when not (B int8 [K,N], scale[n] per column). Two paths:
 *   - transpose_b, M <= 128, K % 64 == 0 (K % 16 == 0 for M <= 4), 16-byte
 *     aligned A and B: the int8 weights are read once, converted to fp16
 *     exactly in registers and multiplied with fp32 sums (dot-product
 *     instructions up to M = 2, and up to M = 4 when K and N are below 8192;
 *     matrix cores otherwise); scale[n] is applied to the sum. No fp16 copy
 *     of the weights. On the matrix cores the sum over K may be split into
 *     up to 8 slices whose fp32 partial sums (a per-stream buffer of
 *     S * M * N floats) a second kernel adds in a fixed order.
 *   - otherwise: the weights are dequantized to fp16 (fp16(q * scale), as the
 *     reference) into a per-stream buffer that grows on demand and is reused,
 *     then multiplied by hipBLASLt with fp32 accumulation.
 * The reference dequantizes into a fresh cudaMalloc'd copy on every call and
 * multiplies with cublasHgemm (matmul.cu:189-244).
 *
 * cuda_gemm_fp16 is C = op(A) @ op(B) through hipBLASLt, fp32 accumulation.
 *
 * Both return 0, or -1 with one line on stderr. They launch on ng_get_stream().
 * Buffers (library workspace, fp16 weight copy, partial sums) belong to a
 * (device, stream) pair; the first call that needs one allocates it and a
 * larger call replaces it with one at least twice its size. Replaced buffers
 * are kept until cuda_shutdown, so a HIP graph that captured an earlier call
 * stays valid. A call that would allocate while the stream is being captured
 * fails instead: make one call of each shape before capture.
 */
#ifndef NG_MATMUL_H
#define NG_MATMUL_H

#include <stdbool.h>

#ifdef __cplusplus
extern "C" {
#endif

/* C[M,N] = op(A) @ op(B), fp16 in and out. A is [M,K] ([K,M] if transpose_a),
 * B is [K,N] ([N,K] if transpose_b). Replaces matmul.h:16-25 (matmul.cu:75-156). */
int cuda_gemm_fp16(void* c, const void* a, const void* b, int M, int K, int N,
                   bool transpose_a, bool transpose_b);

/* C[M,N] = A[M,K] @ (B * scale): A fp16, B int8 [K,N] (or [N,K] when
 * transpose_b), scale fp32 [N], C fp16. Replaces matmul.h:27-38
 * (matmul.cu:189-244). */
int cuda_gemm_int8(void* c, const void* a, const void* b, const void* scale, int M,
                   int K, int N, bool transpose_b);

#ifdef __cplusplus
}
#endif

#endif /* NG_MATMUL_H */
