/* neurogrid_ext.h - entry points of libgpu_engine.so (gfx950 build) that the
 * reference's C ABI does not have. Each one is a fusion or an exported stage
 * of an existing reference path; the comment names the composition it
 * replaces. Return convention as in kernels.h (0 ok, -1 error on stderr).
 */
#ifndef NG_EXT_H
#define NG_EXT_H

#include <stdbool.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Library identification string. */
const char* ng_version(void);

/* Fused RMSNorm + per-token int8 absmax quantisation (fp16 in):
 * y = fp16 RMSNorm(x) as cuda_rmsnorm computes it, then q/scales as
 * cuda_quantize_weights_per_row(q, scales, y, num_tokens, hidden_dim) computes
 * them; y itself is never written. Replaces the composition
 * gpu/cuda/kernels.cu:97-119 followed by gpu/cuda/quantize.cu:320-354.
 * q_out int8 [T, H], scales_out fp32 [T]. */
int ng_rmsnorm_quant_int8(void* q_out, void* scales_out, const void* input, const void* weight,
                          int num_tokens, int hidden_dim, float eps);

/* Residual add + RMSNorm + per-token int8: residual_output as in
 * cuda_add_rmsnorm, then q/scales of the normed row. Replaces
 * gpu/cuda/kernels.cu:237-262 followed by gpu/cuda/quantize.cu:320-354.
 * residual_output may alias residual_input. */
int ng_add_rmsnorm_quant_int8(void* q_out, void* scales_out, void* residual_output, const void* input,
                              const void* residual_input, const void* weight, int num_tokens,
                              int hidden_dim, float eps);

/* bf16 residual add + RMSNorm in one pass, same semantics as cuda_add_rmsnorm.
 * Replaces the bf16 engine's cuda_bf16_add + copy + cuda_bf16_rmsnorm
 * (gpu/engine/layer.cu:1584-1595). */
int ng_bf16_add_rmsnorm(void* normed_output, void* residual_output, const void* input,
                        const void* residual_input, const void* weight, int num_tokens,
                        int hidden_dim, float eps);

/* bf16 SwiGLU in one pass, same semantics as cuda_silu_mul. Replaces the bf16
 * engine's cuda_bf16_silu + cuda_bf16_mul (gpu/engine/layer.cu:1603-1607). */
int ng_bf16_silu_mul(void* output, const void* gate, const void* up, size_t num_elements);

/* RoPE on Q [B, S, num_q_heads, D] and K [B, S, num_kv_heads, D] of the same
 * tokens in one launch, with the semantics of two cuda_rope_with_theta calls
 * sharing `positions` (the pair at gpu/engine/layer.cu:1016,1018). Each
 * token's angles are evaluated once for both tensors. q_out may alias q_in
 * and k_out may alias k_in. The bf16 variant fuses the pair of
 * cuda_bf16_rope_with_theta calls the same way. */
int ng_rope_qk_with_theta(void* q_out, const void* q_in, void* k_out, const void* k_in, const int* positions,
                          int batch_size, int seq_len, int num_q_heads, int num_kv_heads, int head_dim,
                          int rope_style, float rope_theta);
int ng_bf16_rope_qk_with_theta(void* q_out, const void* q_in, void* k_out, const void* k_in, const int* positions,
                               int batch_size, int seq_len, int num_q_heads, int num_kv_heads, int head_dim,
                               int rope_style, float rope_theta);

/* Per-head RMSNorm (QK LayerNorm): x [tokens, heads, head_dim], weight
 * [head_dim] shared by every head; each head's head_dim slice is normalised
 * like a cuda_rmsnorm row. Replaces the engine's static per_head_rmsnorm
 * kernels (gpu/engine/layer.cu:657-701, bf16 1323-1366). output may alias
 * input. */
int ng_per_head_rmsnorm(void* output, const void* input, const void* weight, int num_tokens, int num_heads,
                        int head_dim, float eps);
int ng_bf16_per_head_rmsnorm(void* output, const void* input, const void* weight, int num_tokens,
                             int num_heads, int head_dim, float eps);

/* Per-head RMSNorm of Q and K (weights q_norm_weight, k_norm_weight [head_dim])
 * followed by RoPE on both, in one launch: the same results as
 * ng_per_head_rmsnorm on each tensor and then ng_rope_qk_with_theta. Fuses
 * gpu/engine/layer.cu:998-1018 (QK LayerNorm, then RoPE on Q and K). Outputs
 * may alias their inputs. */
int ng_qk_rmsnorm_rope_with_theta(void* q_out, const void* q_in, void* k_out, const void* k_in,
                                  const void* q_norm_weight, const void* k_norm_weight, const int* positions,
                                  int batch_size, int seq_len, int num_q_heads, int num_kv_heads, int head_dim,
                                  float eps, int rope_style, float rope_theta);
int ng_bf16_qk_rmsnorm_rope_with_theta(void* q_out, const void* q_in, void* k_out, const void* k_in,
                                       const void* q_norm_weight, const void* k_norm_weight, const int* positions,
                                       int batch_size, int seq_len, int num_q_heads, int num_kv_heads,
                                       int head_dim, float eps, int rope_style, float rope_theta);

/* fp32 <-> fp16 on the device (round to nearest even / exact widening): the
 * converters behind gpu/cuda/memory.cu:130-143, exported. */
int ng_fp32_to_fp16(void* output, const void* input, size_t num_elements);
int ng_fp16_to_fp32(void* output, const void* input, size_t num_elements);

/* bf16 [n] -> fp16 [n] with the model loader's truncating rule
 * (pkg/model/loader.go:23-85, ConvertBF16ToFP16, which runs on the host when a
 * bf16 safetensors checkpoint is loaded for the fp16 engine): the same bits,
 * produced on the device. Differs from cuda_bf16_to_fp16 (round to nearest
 * even) only below 2^-14, where it truncates toward zero, and in the NaN
 * payload (always 0x7E00 with the sign). */
int ng_bf16_to_fp16_truncate(void* output, const void* input, size_t num_elements);

/* int8 [rows, cols] -> fp16 [rows, cols], out = fp16(float(q) * scale) with
 * scales[rows] (scale_per_row != 0) or scales[cols]. The dequantisation stage
 * of cuda_gemm_int8, gpu/cuda/matmul.cu:169-187 (dequantize_and_copy), exported
 * so that the caller owns the fp16 buffer instead of a per-call cudaMalloc. */
int cuda_dequantize_weights(void* output, const void* input, const void* scales, int rows, int cols,
                            int scale_per_row);

/* cuda_gather_embeddings with the vocabulary check the Go caller does on the
 * host (pkg/inference/gpu_embeddings.go:52): rows whose id is outside
 * [0, vocab_size) are zero-filled and counted into *d_error_count (device
 * int, not cleared here). */
int ng_gather_embeddings_checked(void* output, const void* embed_table, const int* d_token_ids,
                                 int hidden_size, int num_tokens, int vocab_size, int* d_error_count);

/* cuda_gemm_int8's fused int8 paths (weight streaming for M <= 128, prefill
 * above) without any allocation. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). Arguments as
 * cuda_gemm_int8; results as cuda_gemm_int8 below 4096 rows of A (the same
 * kernels, bit for bit), and the fused prefill kernel's from 4096 rows on,
 * where cuda_gemm_int8 dequantizes and calls hipBLASLt. Shapes: transpose_b,
 * K % 16 == 0 (K % 64 == 0 for 4 < M <= 128), 16-byte aligned A and B; other
 * shapes return -1. The split-K partial sums live in a fixed 64 MiB
 * device array that each GPU the library runs on holds until the process
 * ends; a shape whose partial sums exceed it returns -1. Calls that overlap
 * on one GPU share that array and race. */
int ng_gemm_int8_noalloc(void* c, const void* a, const void* b, const void* scale, int M, int K, int N,
                         bool transpose_b);

/* count (1..4) products that share one A: for i < count,
 *   c[i] = cuda_gemm_int8(c[i], a, b[i], scales[i], M, K, n[i], true)
 * bit for bit (B_i int8 [n[i], K], per-row scales, C_i fp16 [M, n[i]]). The
 * engine's INT8 layer calls cuda_gemm_int8 three times on the same normed rows
 * for q/k/v (gpu/engine/layer.cu:487-501) and twice for gate/up (:575-583).
 * The products that take the same launch shape of cuda_gemm_int8's fused
 * kernels (16-byte aligned A and B, M below 4096) run in one launch of that
 * kernel (plus one launch of the split-K reduction, whose partial sums live
 * in the stream's buffer, as for cuda_gemm_int8); at Mistral-7B's shapes
 * q/k/v together up to 32 tokens, k/v together from 33 to 128, gate/up
 * together up to 128, and on the prefill kernel the products of one tile
 * shape together. Every other product is one cuda_gemm_int8 call. The
 * arrays c, b, scales and n are host arrays. C_i must not overlap A or each
 * other. Returns 0, or -1 (null pointers, count outside 1..4, sizes <= 0, or
 * a failing cuda_gemm_int8). */
int ng_gemm_int8_shared_a(int count, void* const* c, const void* a, const void* const* b,
                          const void* const* scales, const int* n, int M, int K);

/* cuda_rmsnorm(normed, x, norm_weight, M, K, eps) followed by
 * ng_gemm_int8_shared_a(count, c, normed, b, scales, n, M, K), bit for bit:
 * the engine's INT8 layer normalises its input (gpu/engine/layer.cu:467) and
 * then runs q/k/v on it (:487-501). At decode (M <= 2, every product on the
 * GEMV kernel with one shape, at most 1024 of its blocks of 8 rows, K <= 8192,
 * aligned pointers, no output overlapping an input) the norm is folded into
 * the products' launch: each block normalises the rows itself, and normed is
 * still written. Otherwise this is the two calls. Returns 0 or -1. */
int ng_rmsnorm_gemm_int8_shared_a(int count, void* normed, void* const* c, const void* x,
                                  const void* norm_weight, float eps, const void* const* b,
                                  const void* const* scales, const int* n, int M, int K);

/* cuda_add_rmsnorm(normed, residual_out, x, residual_in, norm_weight, M, K,
 * eps) followed by ng_gemm_int8_shared_a(count, c, normed, ...), bit for bit:
 * the residual add and FFN norm of the INT8 layer (gpu/engine/layer.cu:559-570,
 * fused as cuda_add_rmsnorm) and then gate/up (:575-583). Folded into one
 * launch under the conditions above, where also residual_out and normed must
 * not overlap x, residual_in or each other (an in-place call is the two
 * calls). Returns 0 or -1. */
int ng_add_rmsnorm_gemm_int8_shared_a(int count, void* normed, void* residual_out, void* const* c,
                                      const void* x, const void* residual_in, const void* norm_weight,
                                      float eps, const void* const* b, const void* const* scales,
                                      const int* n, int M, int K);

/* The front of the INT8 layer's attention block (gpu/engine/layer.cu:467,
 * 487-501 and the RoPE pair that follows the projections, :1016-1018 in the
 * fp16 layer): ng_rmsnorm_gemm_int8_shared_a(3, normed, {q, k, v}, x,
 * norm_weight, eps, b, scales, {Hq D, Hkv D, Hkv D}, M, hidden), then
 * ng_rope_qk_with_theta(q, q, k, k, positions, 1, M, Hq, Hkv, D, 0,
 * rope_theta): split-half RoPE on q and k in place, one token per row of x
 * with its position. b and scales hold q's, k's and v's. Bit for bit those
 * two calls; where the norm folds into the products' launch (decode, see
 * ng_rmsnorm_gemm_int8_shared_a) and D is a multiple of 8 and at most 256,
 * the rotation runs in that launch too. Returns 0 or -1. */
int ng_rmsnorm_qkv_rope_int8(void* normed, void* q, void* k, void* v, const void* x,
                             const void* norm_weight, float eps, const void* const* b,
                             const void* const* scales, const int* positions, int M, int hidden,
                             int num_q_heads, int num_kv_heads, int head_dim, float rope_theta);

/* The INT8 layer's gate and up projections and SwiGLU (gpu/engine/layer.cu:
 * 575-588: cuda_gemm_int8 twice on one A, then cuda_silu and cuda_mul, which
 * this library's cuda_silu_mul replaces with one rounding): gate and up as
 * ng_gemm_int8_shared_a writes them, then out = cuda_silu_mul(gate, up), bit
 * for bit. With no output overlapping an input or another output (out may
 * be gate or up itself, as the engine's in-place call), one launch computes
 * all three when both products take the GEMV kernel (M <= 4, aligned
 * pointers) or, up to 128 rows, the split kernel with one K slice (wide
 * products, e.g. Mistral-7B's gate/up); with several K slices (e.g.
 * Llama-2-7B's gate/up) one shared split launch and one reduction that also
 * writes SwiGLU; otherwise this is the two calls. B is [N, K] (transpose_b).
 * Returns 0 or -1. */
int ng_gemm_int8_silu_mul(void* out, void* gate, void* up, const void* a, const void* b_gate,
                          const void* scale_gate, const void* b_up, const void* scale_up, int M, int K, int N);

/* The INT8 layer's down projection and final residual add
 * (gpu/engine/layer.cu:593-598): cuda_gemm_int8(c, a, b, scale, M, K, N,
 * true), then cuda_add(out, c, residual, M N), bit for bit. With no output
 * overlapping an input or the other output (out may be c or residual
 * itself): on the GEMV kernel's shapes (M <= 4, aligned pointers) one launch
 * writes both; on the split-K kernel (up to 128 rows) and the prefill kernel
 * (up to 4095) the add runs in the reduction of their K slices. Otherwise
 * this is the two calls. Returns 0 or -1. */
int ng_gemm_int8_add(void* out, void* c, const void* a, const void* b, const void* scale,
                     const void* residual, int M, int K, int N);

#ifdef __cplusplus
}
#endif

#endif /* NG_EXT_H */
