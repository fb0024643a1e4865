/* kernels.h - fp16 per-layer kernels of libgpu_engine.so (gfx950 build).
 *
 * Drop-in replacement for the reference's gpu/cuda/kernels.h (lines 12-89)
 * plus cuda_gather_embeddings, which the reference declares only in
 * gpu/bindings/gpu.h:429-430 (defined at gpu/cuda/kernels.cu:687-708).
 * Every signature, argument meaning and return convention is the
 * reference's: 0 on success, -1 on an invalid argument or a launch error
 * (message on stderr). All launches go to ng_get_stream() (stream.h).
 * Element type is IEEE binary16 unless the name says otherwise.
 */
#ifndef NG_KERNELS_H
#define NG_KERNELS_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* y[t,:] = fp16((x[t,:] * r_t) * w), r_t = 1/sqrt(sum(x^2)/H + eps).
 * Replaces gpu/cuda/kernels.h:12-19 (kernels.cu:97-119). output may alias input. */
int cuda_rmsnorm(void* output, const void* input, const void* weight,
                 int num_tokens, int hidden_dim, float eps);

/* y = fp16(x * sigmoid(x)). Replaces kernels.h:22 (kernels.cu:140-152). */
int cuda_silu(void* output, const void* input, size_t num_elements);

/* c = fp16(a + b). Replaces kernels.h:25 (kernels.cu:298-325). */
int cuda_add(void* c, const void* a, const void* b, size_t num_elements);

/* c = fp16(a * b). Replaces kernels.h:28 (kernels.cu:346-359). */
int cuda_mul(void* c, const void* a, const void* b, size_t num_elements);

/* RoPE pairing styles, values of kernels.h:31-32. */
#define ROPE_STYLE_SPLIT_HALF   0  /* pairs (i, i + D/2): Llama 2, TinyLlama, Mistral */
#define ROPE_STYLE_INTERLEAVED  1  /* pairs (2i, 2i + 1) */

/* Split-half RoPE, theta 10000. Replaces kernels.h:35-43 (kernels.cu:526-537).
 * input/output [batch, seq, num_heads, head_dim]; positions int32 [batch*seq]
 * on the device. output may alias input. */
int cuda_rope(void* output, const void* input, const int* positions,
              int batch_size, int seq_len, int num_heads, int head_dim);

/* RoPE with a style argument, theta 10000. Replaces kernels.h:46-55
 * (kernels.cu:492-523). */
int cuda_rope_styled(void* output, const void* input, const int* positions,
                     int batch_size, int seq_len, int num_heads, int head_dim,
                     int rope_style);

/* RoPE with style and base frequency. Replaces kernels.h:58-68
 * (kernels.cu:540-573). */
int cuda_rope_with_theta(void* output, const void* input, const int* positions,
                         int batch_size, int seq_len, int num_heads, int head_dim,
                         int rope_style, float rope_theta);

/* out = fp16(silu(gate) * up). Replaces kernels.h:71 (kernels.cu:175-188).
 * output may alias gate or up. */
int cuda_silu_mul(void* output, const void* gate, const void* up, size_t num_elements);

/* s = input + residual_input (fp32); residual_output = fp16(s);
 * normed_output = fp16((residual_output * r) * w), r from sum(s^2).
 * Replaces kernels.h:74-83 (kernels.cu:237-262). normed_output may alias
 * input and residual_output may alias residual_input (gpu/engine/layer.cu:1038). */
int cuda_add_rmsnorm(void* normed_output, void* residual_output,
                     const void* input, const void* residual_input,
                     const void* weight, int num_tokens, int hidden_dim, float eps);

/* Row softmax over the last dimension. Replaces kernels.h:86
 * (kernels.cu:633-646); computed with the true row maximum. */
int cuda_softmax(void* output, const void* input, int num_rows, int row_size);

/* y = fp16(x * scale). Replaces kernels.h:89 (kernels.cu:710-723). */
int cuda_scale(void* output, const void* input, float scale, size_t num_elements);

/* out[t,:] = table[ids[t],:], bit copy of 2-byte elements (fp16 or bf16).
 * ids are int32 on the device. Replaces gpu/bindings/gpu.h:429-430
 * (kernels.cu:687-708). Like the reference, ids are not range-checked here;
 * ng_gather_embeddings_checked (neurogrid_ext.h) checks them. */
int cuda_gather_embeddings(void* output, const void* embed_table,
                           const int* d_token_ids, int hidden_size, int num_tokens);

#ifdef __cplusplus
}
#endif

#endif /* NG_KERNELS_H */
