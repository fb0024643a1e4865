// gather.hip - embedding gather: out[t, :] = table[ids[t], :], a bit copy of
// 2-byte elements (fp16 or bf16 alike).
//
// Reference: gpu/cuda/kernels.cu:669-708 (one thread per element, integer
// div/mod per element). Here one wave copies one row with 16-byte vectors;
// the id is read once per row into a scalar register. Table reads keep the
// default cache policy (hot ids repeat); output stores are non-temporal.
#include "ng_common.hpp"

namespace ng {

constexpr int kGatherThreads = 256;
constexpr int kGatherRowsPerBlock = kGatherThreads / kWave;
constexpr int kGatherChunk = 8;  // 16-byte vectors per lane loaded before any store

// vocab > 0 turns on the range check: rows whose id is outside [0, vocab)
// are zero-filled and counted in *bad. Each chunk of up to 8 vectors per lane
// is loaded in full before it is stored (unconditional loads from clamped
// indices, predicated stores), so a row of up to 1024 elements is one load
// phase and one store phase.
__global__ __launch_bounds__(kGatherThreads) void gather_vec_kernel(void* out, const void* table, const int* ids,
                                                                   int T, int nvec, int vocab, int* bad) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * kGatherRowsPerBlock + (threadIdx.x >> 6);
    if (t >= T) return;
    const int id = __builtin_amdgcn_readfirstlane(ids[t]);
    u32x4* dst = reinterpret_cast<u32x4*>(out) + static_cast<size_t>(t) * nvec;
    if (vocab > 0 && (id < 0 || id >= vocab)) {
        for (int v = lane; v < nvec; v += kWave) st16_stream(dst + v, u32x4{0, 0, 0, 0});
        if (lane == 0) atomicAdd(bad, 1);
        return;
    }
    const u32x4* src = reinterpret_cast<const u32x4*>(table) + static_cast<size_t>(id) * nvec;
    for (int v0 = 0; v0 < nvec; v0 += kWave * kGatherChunk) {
        u32x4 r[kGatherChunk];
#pragma unroll
        for (int k = 0; k < kGatherChunk; ++k) {
            const int v = v0 + lane + k * kWave;
            r[k] = ld16(src + (v < nvec ? v : nvec - 1));
        }
#pragma unroll
        for (int k = 0; k < kGatherChunk; ++k) {
            const int v = v0 + lane + k * kWave;
            if (v < nvec) st16_stream(dst + v, r[k]);
        }
    }
}

__global__ __launch_bounds__(kGatherThreads) void gather_scalar_kernel(uint16_t* out, const uint16_t* table,
                                                                      const int* ids, int H, int T, int vocab,
                                                                      int* bad) {
    const int t = blockIdx.x;
    if (t >= T) return;
    const int id = ids[t];
    uint16_t* dst = out + static_cast<size_t>(t) * H;
    if (vocab > 0 && (id < 0 || id >= vocab)) {
        for (int i = threadIdx.x; i < H; i += kGatherThreads) dst[i] = 0;
        if (threadIdx.x == 0) atomicAdd(bad, 1);
        return;
    }
    const uint16_t* src = table + static_cast<size_t>(id) * H;
    for (int i = threadIdx.x; i < H; i += kGatherThreads) dst[i] = src[i];
}

static int launch_gather(const char* name, void* output, const void* table, const int* ids, int H, int T,
                         int vocab, int* bad) {
    NG_REQUIRE(output && table && ids, "%s: null pointer", name);
    NG_REQUIRE(H > 0 && T > 0, "%s: hidden_size=%d num_tokens=%d must be > 0", name, H, T);
    if (H % 8 == 0 && aligned16(output) && aligned16(table)) {
        const unsigned blocks = static_cast<unsigned>((T + kGatherRowsPerBlock - 1) / kGatherRowsPerBlock);
        gather_vec_kernel<<<dim3(blocks), dim3(kGatherThreads), 0, stream()>>>(output, table, ids, T, H / 8, vocab,
                                                                             bad);
    } else {
        gather_scalar_kernel<<<dim3(T), dim3(kGatherThreads), 0, stream()>>>(
            static_cast<uint16_t*>(output), static_cast<const uint16_t*>(table), ids, H, T, vocab, bad);
    }
    NG_CHECK_LAUNCH(name);
    return 0;
}

}  // namespace ng

using namespace ng;

extern "C" int cuda_gather_embeddings(void* output, const void* embed_table, const int* d_token_ids,
                                      int hidden_size, int num_tokens) {
    return launch_gather("cuda_gather_embeddings", output, embed_table, d_token_ids, hidden_size, num_tokens, 0,
                         nullptr);
}

extern "C" int ng_gather_embeddings_checked(void* output, const void* embed_table, const int* d_token_ids,
                                            int hidden_size, int num_tokens, int vocab_size, int* d_error_count) {
    NG_REQUIRE(vocab_size > 0, "ng_gather_embeddings_checked: vocab_size=%d must be > 0", vocab_size);
    NG_REQUIRE(d_error_count, "ng_gather_embeddings_checked: null error counter");
    return launch_gather("ng_gather_embeddings_checked", output, embed_table, d_token_ids, hidden_size, num_tokens,
                         vocab_size, d_error_count);
}
