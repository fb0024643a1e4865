// rope.hip - rotary position embedding on [batch, seq, heads, head_dim].
//
// Semantics (reference: gpu/cuda/kernels.cu:431-489, bf16_utils.cu:330-378):
//   inv_i = 1 / powf(theta, (2 i) / D)         i < D/2, computed on the host
//   a     = float(pos[t]) * inv_i               one fp32 rounding
//   (c, s)= (cos a, sin a)                      accurate sincosf
//   x1' = x1 c - x2 s,  x2' = x1 s + x2 c       rounded once to the element type
//   split-half pairs (i, i + D/2); interleaved pairs (2i, 2i + 1)
//
// The angle depends on (token, pair) only. A workgroup takes a tile of tokens,
// evaluates each of its tile * D/2 (cos, sin) pairs once into LDS, then
// rotates every head of those tokens with 16-byte vector accesses; the
// reference evaluates powf/sincos again for every head.
#include "ng_common.hpp"

#include <math.h>

#include <mutex>
#include <unordered_map>
#include <vector>

namespace ng {

constexpr int kRopeThreads = 256;
constexpr int kRopeMaxHalf = 128;  // D <= 256

struct RopeArgs {
    void* out;
    const void* in;
    const int* pos;
    int T;             // tokens
    int nh;            // heads
    int D;             // head_dim
    int half;          // D / 2
    int upt;           // work units per token
    int tb;            // tokens per workgroup
    FastDiv div_upt;   // divide by units per token
    FastDiv div_uph;   // divide by units per head
    float inv_freq[kRopeMaxHalf];
};

// Split-half vector unit: pairs [8j, 8j+8) of one head, i.e. the 16-byte
// vectors at offsets 8j and D/2 + 8j. Interleaved vector unit: the 16-byte
// vector at offset 8j, holding pairs [4j, 4j+4).
template <typename T, int STYLE>
__global__ __launch_bounds__(kRopeThreads) void rope_vec_kernel(RopeArgs a) {
    extern __shared__ float2 cs[];  // [tb][half]
    const int t0 = blockIdx.x * a.tb;
    const int ncs = a.tb * a.half;
    for (int idx = threadIdx.x; idx < ncs; idx += kRopeThreads) {
        const int tl = idx / a.half;
        const int i = idx - tl * a.half;
        const int t = t0 + tl;
        float c = 1.0f, s = 0.0f;
        if (t < a.T) {
            const float ang = static_cast<float>(a.pos[t]) * a.inv_freq[i];
            sincosf(ang, &s, &c);
        }
        cs[idx] = make_float2(c, s);
    }
    __syncthreads();

    const int units = a.tb * a.upt;
    const uint16_t* in = static_cast<const uint16_t*>(a.in);
    uint16_t* out = static_cast<uint16_t*>(a.out);
    for (int u = threadIdx.x; u < units; u += kRopeThreads) {
        const int tl = static_cast<int>(fdiv(static_cast<uint32_t>(u), a.div_upt));
        const int t = t0 + tl;
        if (t >= a.T) break;
        const int rem = u - tl * a.upt;
        const int h = static_cast<int>(fdiv(static_cast<uint32_t>(rem), a.div_uph));
        const int j = rem - h * static_cast<int>(a.div_uph.d);
        const size_t base = (static_cast<size_t>(t) * a.nh + h) * a.D;
        const float2* c = cs + tl * a.half;
        if (STYLE == 0) {
            const u32x4 v1 = ld16(in + base + 8 * j);
            const u32x4 v2 = ld16(in + base + a.half + 8 * j);
            float x1[8], x2[8], y1[8], y2[8];
            unpack8<T>(v1, x1);
            unpack8<T>(v2, x2);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float2 k = c[8 * j + e];
                y1[e] = x1[e] * k.x - x2[e] * k.y;
                y2[e] = x1[e] * k.y + x2[e] * k.x;
            }
            st16(out + base + 8 * j, pack8<T>(y1));
            st16(out + base + a.half + 8 * j, pack8<T>(y2));
        } else {
            const u32x4 v = ld16(in + base + 8 * j);
            float x[8], y[8];
            unpack8<T>(v, x);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float2 k = c[4 * j + e];
                y[2 * e] = x[2 * e] * k.x - x[2 * e + 1] * k.y;
                y[2 * e + 1] = x[2 * e] * k.y + x[2 * e + 1] * k.x;
            }
            st16(out + base + 8 * j, pack8<T>(y));
        }
    }
}

// Any head_dim and alignment: one thread per (token, head, pair).
template <typename T>
__global__ __launch_bounds__(kRopeThreads) void rope_scalar_kernel(RopeArgs a, int style) {
    const size_t npairs = static_cast<size_t>(a.T) * a.nh * a.half;
    const uint16_t* in = static_cast<const uint16_t*>(a.in);
    uint16_t* out = static_cast<uint16_t*>(a.out);
    const size_t stride = static_cast<size_t>(gridDim.x) * kRopeThreads;
    for (size_t p = static_cast<size_t>(blockIdx.x) * kRopeThreads + threadIdx.x; p < npairs; p += stride) {
        const int i = static_cast<int>(p % a.half);
        const size_t th = p / a.half;  // token * nh + head
        const int t = static_cast<int>(th / a.nh);
        const size_t base = th * a.D;
        const size_t i1 = style == 1 ? base + 2 * i : base + i;
        const size_t i2 = style == 1 ? base + 2 * i + 1 : base + i + a.half;
        float s, c;
        sincosf(static_cast<float>(a.pos[t]) * a.inv_freq[i], &s, &c);
        const float x1 = to_f32<T>(in[i1]), x2 = to_f32<T>(in[i2]);
        const float y1 = x1 * c - x2 * s;
        const float y2 = x1 * s + x2 * c;
        out[i1] = from_f32<T>(y1);
        out[i2] = from_f32<T>(y2);
    }
}

// inv_freq tables, cached per (theta bits, head_dim): 64 powf calls per miss.
static void fill_inv_freq(float theta, int D, float* dst) {
    static std::mutex mu;
    static std::unordered_map<uint64_t, std::vector<float>> cache;
    const uint64_t key = (static_cast<uint64_t>(__builtin_bit_cast(uint32_t, theta)) << 32) |
                         static_cast<uint32_t>(D);
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it == cache.end()) {
        std::vector<float> v(D / 2);
        for (int i = 0; i < D / 2; ++i) {
            const float expo = (2.0f * static_cast<float>(i)) / static_cast<float>(D);
            v[i] = 1.0f / powf(theta, expo);
        }
        it = cache.emplace(key, std::move(v)).first;
    }
    for (int i = 0; i < D / 2; ++i) dst[i] = it->second[i];
}

template <typename T>
static int launch_rope(const char* name, void* output, const void* input, const int* positions,
                       int batch_size, int seq_len, int num_heads, int head_dim, int style, float theta) {
    NG_REQUIRE(output && input && positions, "%s: null pointer", name);
    NG_REQUIRE(batch_size > 0 && seq_len > 0 && num_heads > 0, "%s: batch=%d seq=%d heads=%d must be > 0",
               name, batch_size, seq_len, num_heads);
    NG_REQUIRE(head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 2 * kRopeMaxHalf,
               "%s: head_dim=%d must be even and in [2, %d]", name, head_dim, 2 * kRopeMaxHalf);
    // As in the reference (kernels.cu:469), every style other than 1 pairs split-half.
    style = style == 1 ? 1 : 0;
    const long long T64 = static_cast<long long>(batch_size) * seq_len;
    NG_REQUIRE(T64 * num_heads * head_dim < (1ll << 31), "%s: tensor too large", name);

    RopeArgs a{};
    a.out = output;
    a.in = input;
    a.pos = positions;
    a.T = static_cast<int>(T64);
    a.nh = num_heads;
    a.D = head_dim;
    a.half = head_dim / 2;
    fill_inv_freq(theta, head_dim, a.inv_freq);

    const bool aligned = aligned16(output) && aligned16(input);
    const bool vec = aligned && ((style == 0 && head_dim % 16 == 0) || (style == 1 && head_dim % 8 == 0));
    if (vec) {
        const int uph = style == 0 ? head_dim / 16 : head_dim / 8;
        a.upt = num_heads * uph;
        // About 1024 units per workgroup; at least one token; LDS <= 32 KiB.
        int tb = (1024 + a.upt - 1) / a.upt;
        const int max_tb_lds = (32 * 1024) / (a.half * static_cast<int>(sizeof(float2)));
        if (tb > max_tb_lds) tb = max_tb_lds;
        if (tb < 1) tb = 1;
        if (tb > a.T) tb = a.T;
        a.tb = tb;
        a.div_upt = make_fastdiv(static_cast<uint32_t>(a.upt));
        a.div_uph = make_fastdiv(static_cast<uint32_t>(uph));
        const unsigned blocks = static_cast<unsigned>((a.T + tb - 1) / tb);
        const size_t lds = static_cast<size_t>(tb) * a.half * sizeof(float2);
        if (style == 0)
            rope_vec_kernel<T, 0><<<dim3(blocks), dim3(kRopeThreads), lds, stream()>>>(a);
        else
            rope_vec_kernel<T, 1><<<dim3(blocks), dim3(kRopeThreads), lds, stream()>>>(a);
    } else {
        const size_t npairs = static_cast<size_t>(a.T) * num_heads * a.half;
        size_t blocks = (npairs + kRopeThreads - 1) / kRopeThreads;
        if (blocks > 65536) blocks = 65536;
        rope_scalar_kernel<T><<<dim3(static_cast<unsigned>(blocks)), dim3(kRopeThreads), 0, stream()>>>(a, style);
    }
    NG_CHECK_LAUNCH(name);
    return 0;
}

}  // namespace ng

using namespace ng;

extern "C" int cuda_rope_with_theta(void* output, const void* input, const int* positions, int batch_size,
                                    int seq_len, int num_heads, int head_dim, int rope_style, float rope_theta) {
    return launch_rope<f16>("cuda_rope_with_theta", output, input, positions, batch_size, seq_len, num_heads,
                            head_dim, rope_style, rope_theta);
}

extern "C" int cuda_rope_styled(void* output, const void* input, const int* positions, int batch_size,
                                int seq_len, int num_heads, int head_dim, int rope_style) {
    return launch_rope<f16>("cuda_rope_styled", output, input, positions, batch_size, seq_len, num_heads,
                            head_dim, rope_style, 10000.0f);
}

extern "C" int cuda_rope(void* output, const void* input, const int* positions, int batch_size, int seq_len,
                         int num_heads, int head_dim) {
    return launch_rope<f16>("cuda_rope", output, input, positions, batch_size, seq_len, num_heads, head_dim,
                            0, 10000.0f);
}

extern "C" int cuda_bf16_rope_with_theta(void* output, const void* input, const int* positions, int batch_size,
                                         int seq_len, int num_heads, int head_dim, int rope_style,
                                         float rope_theta) {
    return launch_rope<bf16>("cuda_bf16_rope_with_theta", output, input, positions, batch_size, seq_len,
                             num_heads, head_dim, rope_style, rope_theta);
}
