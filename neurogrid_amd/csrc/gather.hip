// gather.hip - embedding gather: out[t, :] = table[ids[t], :], a bit copy of
// 2-byte elements (fp16 or bf16 alike).
//
// Reference: gpu/cuda/kernels.cu:669-708 (one thread per element, integer
// div/mod per element). Here a wave copies whole rows with 16-byte vectors;
// each id is read once into a scalar register. Table reads keep the default
// cache policy (hot ids repeat); output stores are non-temporal.
#include "ng_common.hpp"

#include <type_traits>

namespace ng {

constexpr int kGatherThreads = 256;
constexpr int kGatherRowsPerBlock = kGatherThreads / kWave;
constexpr int kGatherChunk = 8;  // 16-byte vectors per lane loaded before any store

// vocab > 0 turns on the range check: rows whose id is outside [0, vocab)
// are zero-filled and counted in *bad.
//
// gather_rows_kernel: a wave copies R rows of up to 64 V vectors. It reads
// the R ids (the wave index is marked uniform, so the ids arrive through
// scalar loads, all issued before the first is waited on: 0.7% faster at
// Mistral-7B prefill, 1.5% with Zipf ids at Mistral-Nemo, than vector loads
// and readfirstlane), issues every load of the R rows (unconditional, from
// clamped indices), and only then stores the rows in turn, so the stores of
// the first rows overlap the arrival of the later ones. Measured on MI355X at
// T = 4096, H = 4096 with uniform ids: 12.3 us with R = 4 against 13.5 us
// for one row per wave; one row per wave stays best at T = 2048, H = 5120
// (6.1 us with Zipf ids). Table reads keep the default cache policy: with
// Zipf-distributed ids hot rows come from the cache (non-temporal loads
// were 3% faster with uniform ids and 15% slower with Zipf ids).
template <int R, int V, bool CHECK>
__global__ __launch_bounds__(kGatherThreads) void gather_rows_kernel(void* __restrict__ out,
                                                                    const void* __restrict__ table,
                                                                    const int* __restrict__ ids, int T, int nvec,
                                                                    int vocab, int* __restrict__ bad) {
    const int lane = threadIdx.x & 63;
    const int t0 = R * (blockIdx.x * kGatherRowsPerBlock + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
    if (t0 >= T) return;
    const u32x4* src[R];
    bool valid[R];
    int idr[R];
#pragma unroll
    for (int q = 0; q < R; ++q) idr[q] = ids[min(t0 + q, T - 1)];
#pragma unroll
    for (int q = 0; q < R; ++q) {
        const int id = __builtin_amdgcn_readfirstlane(idr[q]);
        valid[q] = !CHECK || (id >= 0 && id < vocab);
        src[q] = reinterpret_cast<const u32x4*>(table) + static_cast<size_t>(valid[q] ? id : 0) * nvec;
    }
    u32x4 r[R][V];
#pragma unroll
    for (int q = 0; q < R; ++q)
#pragma unroll
        for (int k = 0; k < V; ++k) {
            const int v = lane + k * kWave;
            r[q][k] = ld16(src[q] + (v < nvec ? v : nvec - 1));
        }
#pragma unroll
    for (int q = 0; q < R; ++q) {
        if (t0 + q >= T) break;
        u32x4* dst = reinterpret_cast<u32x4*>(out) + static_cast<size_t>(t0 + q) * nvec;
        if (CHECK && !valid[q] && lane == 0) atomicAdd(bad, 1);
#pragma unroll
        for (int k = 0; k < V; ++k) {
            const int v = lane + k * kWave;
            if (v < nvec) st16_stream(dst + v, !CHECK || valid[q] ? r[q][k] : u32x4{0, 0, 0, 0});
        }
    }
}

// Rows of more than 640 vectors: chunks of up to 8 vectors per lane, each
// loaded in full before it is stored.
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
    const int nvec = H / 8;
    if (H % 8 == 0 && aligned16(output) && aligned16(table) && nvec <= 640) {
        // Four rows per wave for rows of up to 512 vectors when that still
        // leaves 1024 waves or more; otherwise one.
        const int R = nvec <= 512 && T >= 4096 ? 4 : 1;
        const unsigned blocks = static_cast<unsigned>((T + R * kGatherRowsPerBlock - 1) / (R * kGatherRowsPerBlock));
        const int V = (nvec + kWave - 1) / kWave;
        auto go = [&](auto check) {
            constexpr bool C = decltype(check)::value;
            auto run = [&](auto kern) {
                kern<<<dim3(blocks), dim3(kGatherThreads), 0, stream()>>>(output, table, ids, T, nvec, vocab, bad);
            };
            if (R == 4) {
                if (V <= 2) run(gather_rows_kernel<4, 2, C>);
                else if (V <= 4) run(gather_rows_kernel<4, 4, C>);
                else run(gather_rows_kernel<4, 8, C>);
            } else {
                if (V <= 2) run(gather_rows_kernel<1, 2, C>);
                else if (V <= 4) run(gather_rows_kernel<1, 4, C>);
                else if (V <= 8) run(gather_rows_kernel<1, 8, C>);
                else run(gather_rows_kernel<1, 10, C>);
            }
        };
        if (vocab > 0) go(std::true_type{});
        else go(std::false_type{});
    } else if (H % 8 == 0 && aligned16(output) && aligned16(table)) {
        const unsigned blocks = static_cast<unsigned>((T + kGatherRowsPerBlock - 1) / kGatherRowsPerBlock);
        gather_vec_kernel<<<dim3(blocks), dim3(kGatherThreads), 0, stream()>>>(output, table, ids, T, nvec, vocab,
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
