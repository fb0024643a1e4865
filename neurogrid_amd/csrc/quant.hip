// quant.hip - per-tensor and per-column int8 absmax quantisation, and
// int8 -> fp16 dequantisation (per tensor, per row, per column).
//
// Quantisation rule (reference: gpu/cuda/quantize.cu:59-95, 189-231, with
// half-to-even rounding): m = max|x| over the non-NaN elements (the
// reference's fmaxf reduction skips NaNs), scale = m / 127 (1 if that is 0),
// q = fmaxf(-127, fminf(127, rint(x / scale))), IEEE division; a NaN element
// gets +127.
// Dequantisation (quantize.cu:147-158, matmul.cu:169-187):
// out = RN_f16(RN_f32(float(q) * scale)).
//
// The reference's per-tensor path allocates a device word and reads the
// maximum back to the host (quantize.cu:104-128). Here the maximum lives in
// the caller's scale word itself: zero it, atomicMax the fp16 magnitude
// patterns into it, quantise, then overwrite it with the scale - four
// launches in stream order, no allocation, no host synchronisation.
// Per-column quantisation uses the caller's scales[N] the same way.
#include "ng_common.hpp"

namespace ng {

constexpr int kQThreads = 256;

__device__ __forceinline__ float scale_from_bits(uint32_t mbits) {
    const float m = to_f32<f16>(static_cast<uint16_t>(mbits));
    const float s = m / 127.0f;
    return s == 0.0f ? 1.0f : s;
}

// q = clamp(rint(RN(v / scale)), -127, 127) without a division (qcode_int).
__device__ __forceinline__ int qcode(float v, float scale, float inv) { return qcode_int(v, scale, inv); }

__global__ void fill_u32_kernel(uint32_t* p, size_t n, uint32_t v) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}

// ---- per tensor --------------------------------------------------------------
constexpr int kAbsLoads = 4;

__global__ __launch_bounds__(kQThreads) void tensor_absmax_kernel(uint32_t* mx_out, const uint16_t* x, size_t n,
                                                                  int vec) {
    __shared__ uint32_t s_max[kQThreads / kWave];
    const size_t stride = static_cast<size_t>(gridDim.x) * kQThreads;
    const size_t t0 = static_cast<size_t>(blockIdx.x) * kQThreads + threadIdx.x;
    uint32_t m = 0;
    size_t done = 0;
    auto fold = [&m](const u32x4 v) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t lo = absbits_nonan<f16>(static_cast<uint16_t>(v[k]));
            const uint32_t hi = absbits_nonan<f16>(static_cast<uint16_t>(v[k] >> 16));
            m = m > lo ? m : lo;
            m = m > hi ? m : hi;
        }
    };
    if (vec) {
        // kAbsLoads vectors per thread per pass, all requested before any is
        // folded: with one at a time each wave kept a single load in flight.
        // Measured on MI355X for 2^27 elements: the whole per-tensor call
        // 124.5 us against 129.8 us (8 loads: 125.7 us).
        const size_t nvec = n / 8;
        size_t i = t0;
        for (; i + (kAbsLoads - 1) * stride < nvec; i += kAbsLoads * stride) {
            u32x4 v[kAbsLoads];
#pragma unroll
            for (int u = 0; u < kAbsLoads; ++u) v[u] = ld16_stream(x + (i + u * stride) * 8);
#pragma unroll
            for (int u = 0; u < kAbsLoads; ++u) fold(v[u]);
        }
        for (; i < nvec; i += stride) fold(ld16_stream(x + i * 8));
        done = nvec * 8;
    }
    for (size_t i = done + t0; i < n; i += stride) {
        const uint32_t b = absbits_nonan<f16>(x[i]);
        m = m > b ? m : b;
    }
    m = wave_max_u32(m);
    if ((threadIdx.x & 63) == 0) s_max[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int j = 1; j < kQThreads / kWave; ++j) m = m > s_max[j] ? m : s_max[j];
        atomicMax(mx_out, m);
    }
}

__global__ __launch_bounds__(kQThreads) void tensor_quant_kernel(int8_t* q, const uint16_t* x, const uint32_t* mx,
                                                                 size_t n, int vec) {
    const float scale = scale_from_bits(*mx);
    const float inv = 1.0f / scale;
    const size_t stride = static_cast<size_t>(gridDim.x) * kQThreads;
    const size_t t0 = static_cast<size_t>(blockIdx.x) * kQThreads + threadIdx.x;
    size_t done = 0;
    if (vec) {
        const size_t nvec = n / 8;
        for (size_t i = t0; i < nvec; i += stride) {
            float f[8];
            unpack8<f16>(ld16_stream(x + i * 8), f);
            uint32_t c[2] = {0, 0};
#pragma unroll
            for (int e = 0; e < 8; ++e)
                c[e >> 2] |= (static_cast<uint32_t>(qcode(f[e], scale, inv)) & 0xffu) << ((e & 3) * 8);
            *reinterpret_cast<u32x2*>(q + i * 8) = u32x2{c[0], c[1]};
        }
        done = nvec * 8;
    }
    for (size_t i = done + t0; i < n; i += stride) q[i] = static_cast<int8_t>(qcode(to_f32<f16>(x[i]), scale, inv));
}

__global__ void tensor_scale_finalize_kernel(float* scale) {
    const uint32_t mbits = *reinterpret_cast<const uint32_t*>(scale);
    *scale = scale_from_bits(mbits);
}

// ---- per column of [K, N] ------------------------------------------------------
// Thread = one column (scalar) or one group of 8 columns (vector), over a
// chunk of rows; the chunk maximum is folded into colmax[N] with atomicMax.
__global__ __launch_bounds__(kQThreads) void col_absmax_kernel(uint32_t* colmax, const uint16_t* x, int K, int N,
                                                               int rows_per_chunk, int vec) {
    const int r0 = blockIdx.y * rows_per_chunk;
    const int r1 = min(K, r0 + rows_per_chunk);
    if (vec) {
        const int cv = blockIdx.x * kQThreads + threadIdx.x;
        if (cv >= N / 8) return;
        uint32_t m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int r = r0; r < r1; ++r) {
            const u32x4 v = ld16(x + static_cast<size_t>(r) * N + cv * 8);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t b = absbits_nonan<f16>(lane16(v, e));
                m[e] = m[e] > b ? m[e] : b;
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) atomicMax(colmax + cv * 8 + e, m[e]);
    } else {
        const int c = blockIdx.x * kQThreads + threadIdx.x;
        if (c >= N) return;
        uint32_t m = 0;
        for (int r = r0; r < r1; ++r) {
            const uint32_t b = absbits_nonan<f16>(x[static_cast<size_t>(r) * N + c]);
            m = m > b ? m : b;
        }
        atomicMax(colmax + c, m);
    }
}

__global__ __launch_bounds__(kQThreads) void col_quant_kernel(int8_t* q, const uint16_t* x, const uint32_t* colmax,
                                                              int K, int N, int vec) {
    if (vec) {
        const int cv = blockIdx.x * kQThreads + threadIdx.x;
        if (cv >= N / 8) return;
        float sc[8], inv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            sc[e] = scale_from_bits(colmax[cv * 8 + e]);
            inv[e] = 1.0f / sc[e];
        }
        for (int r = blockIdx.y; r < K; r += gridDim.y) {
            float f[8];
            unpack8<f16>(ld16(x + static_cast<size_t>(r) * N + cv * 8), f);
            uint32_t c[2] = {0, 0};
#pragma unroll
            for (int e = 0; e < 8; ++e)
                c[e >> 2] |= (static_cast<uint32_t>(qcode(f[e], sc[e], inv[e])) & 0xffu) << ((e & 3) * 8);
            *reinterpret_cast<u32x2*>(q + static_cast<size_t>(r) * N + cv * 8) = u32x2{c[0], c[1]};
        }
    } else {
        const int c = blockIdx.x * kQThreads + threadIdx.x;
        if (c >= N) return;
        const float sc = scale_from_bits(colmax[c]);
        const float inv = 1.0f / sc;
        for (int r = blockIdx.y; r < K; r += gridDim.y) {
            const size_t i = static_cast<size_t>(r) * N + c;
            q[i] = static_cast<int8_t>(qcode(to_f32<f16>(x[i]), sc, inv));
        }
    }
}

__global__ void col_scale_finalize_kernel(float* scales, int N) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c < N) scales[c] = scale_from_bits(reinterpret_cast<const uint32_t*>(scales)[c]);
}

// ---- dequantisation ----------------------------------------------------------
enum DqMode : int { DQ_ROW = 0, DQ_COL = 1, DQ_TENSOR = 2 };

// Vector path: one 16-byte int8 load -> two 16-byte fp16 stores, one group
// of 16 codes per thread over a flat grid (every group of the matrix has its
// own thread). groups_per_row = cols / 16; the row of group g is
// g / groups_per_row (a run-time-constant division).
template <int MODE>
__global__ __launch_bounds__(kQThreads) void dequant_vec_kernel(uint16_t* out, const int8_t* q, const float* scales,
                                                                uint32_t ngroups, FastDiv gpr) {
    const uint32_t g = blockIdx.x * kQThreads + threadIdx.x;
    if (g >= ngroups) return;
    const size_t e0 = static_cast<size_t>(g) * 16;
    const u32x4 v = ld16_stream(q + e0);
    float s[16];
    if (MODE == DQ_ROW) {
        const float rs = scales[fdiv(g, gpr)];
#pragma unroll
        for (int e = 0; e < 16; ++e) s[e] = rs;
    } else if (MODE == DQ_COL) {
        const uint32_t cg = g - fdiv(g, gpr) * gpr.d;  // group within the row
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const u32x4 sv = ld16(scales + cg * 16 + 4 * k);
#pragma unroll
            for (int e = 0; e < 4; ++e) s[4 * k + e] = as_float(sv[e]);
        }
    } else {
        const float ts = scales[0];
#pragma unroll
        for (int e = 0; e < 16; ++e) s[e] = ts;
    }
    float lo[8], hi[8];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int8_t c = static_cast<int8_t>((v[e >> 2] >> ((e & 3) * 8)) & 0xffu);
        const float f = static_cast<float>(c) * s[e];
        if (e < 8) lo[e] = f; else hi[e - 8] = f;
    }
    st16_stream(out + e0, pack8<f16>(lo));
    st16_stream(out + e0 + 8, pack8<f16>(hi));
}

// Chunked path for rows that are a multiple of 512 codes. A chunk is 512
// consecutive codes of one row; lane l of a wave owns codes [8l, 8l + 8) of
// each of its DQ_CHUNKS chunks: one 8-byte load and one 16-byte store per
// chunk, so every load instruction reads 512 contiguous bytes and every store
// instruction writes 1 KiB of whole cache lines. (Writing 16 codes per lane,
// i.e. two 16-byte stores 32 bytes apart, leaves every line half-written by
// each instruction; measured on MI355X that costs 27% at [14336, 4096].)
constexpr int kDqChunks = 2;

template <int MODE>
__global__ __launch_bounds__(kQThreads) void dequant_chunk_kernel(uint16_t* out, const int8_t* q, const float* scales,
                                                                  uint32_t nchunks, FastDiv chunks_per_row) {
    const int lane = threadIdx.x & 63;
    const uint32_t wv = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    u32x2 v[kDqChunks];
    uint32_t ch[kDqChunks];
#pragma unroll
    for (int c = 0; c < kDqChunks; ++c) {
        ch[c] = wv * kDqChunks + c;
        const uint32_t cc = ch[c] < nchunks ? ch[c] : nchunks - 1;
        v[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(q + static_cast<size_t>(cc) * 512 + 8 * lane));
    }
#pragma unroll
    for (int c = 0; c < kDqChunks; ++c) {
        if (ch[c] >= nchunks) break;
        float s[8];
        if (MODE == DQ_ROW) {
            const float rs = scales[fdiv(ch[c], chunks_per_row)];
#pragma unroll
            for (int e = 0; e < 8; ++e) s[e] = rs;
        } else if (MODE == DQ_COL) {
            const uint32_t col = (ch[c] - fdiv(ch[c], chunks_per_row) * chunks_per_row.d) * 512 + 8 * lane;
            const u32x4 s0 = ld16(scales + col), s1 = ld16(scales + col + 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                s[e] = as_float(s0[e]);
                s[4 + e] = as_float(s1[e]);
            }
        } else {
            const float ts = scales[0];
#pragma unroll
            for (int e = 0; e < 8; ++e) s[e] = ts;
        }
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = static_cast<float>(static_cast<int8_t>((v[c][e >> 2] >> ((e & 3) * 8)) & 0xffu)) * s[e];
        st16_stream(out + static_cast<size_t>(ch[c]) * 512 + 8 * lane, pack8<f16>(f));
    }
}

template <int MODE>
__global__ __launch_bounds__(kQThreads) void dequant_scalar_kernel(uint16_t* out, const int8_t* q,
                                                                   const float* scales, size_t n, int cols) {
    const size_t stride = static_cast<size_t>(gridDim.x) * kQThreads;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kQThreads + threadIdx.x; i < n; i += stride) {
        float s;
        if (MODE == DQ_ROW) s = scales[i / cols];
        else if (MODE == DQ_COL) s = scales[i % cols];
        else s = scales[0];
        out[i] = from_f32<f16>(static_cast<float>(q[i]) * s);
    }
}

template <int MODE>
static int launch_dequant(const char* name, void* out, const void* q, const void* scales, size_t rows, size_t cols) {
    const size_t n = rows * cols;
    const bool vec = cols % 16 == 0 && aligned16(out) && aligned16(q) && (MODE != DQ_COL || aligned16(scales)) &&
                     n / 16 < (1ull << 32) && cols / 16 < (1ull << 31);
    if (vec && cols % 512 == 0 && aligned8(q) && n / 512 < (1ull << 32)) {
        const uint32_t nchunks = static_cast<uint32_t>(n / 512);
        const uint32_t waves = (nchunks + kDqChunks - 1) / kDqChunks;
        // One wave per workgroup: 28.7 vs 30.2 us at [14336, 4096] with four.
        const unsigned blocks = waves;
        dequant_chunk_kernel<MODE><<<dim3(blocks), dim3(kWave), 0, stream()>>>(
            static_cast<uint16_t*>(out), static_cast<const int8_t*>(q), static_cast<const float*>(scales), nchunks,
            make_fastdiv(static_cast<uint32_t>(cols / 512)));
    } else if (vec) {
        const uint32_t ngroups = static_cast<uint32_t>(n / 16);
        const unsigned blocks = static_cast<unsigned>((ngroups + kQThreads - 1) / kQThreads);
        dequant_vec_kernel<MODE><<<dim3(blocks), dim3(kQThreads), 0, stream()>>>(
            static_cast<uint16_t*>(out), static_cast<const int8_t*>(q), static_cast<const float*>(scales), ngroups,
            make_fastdiv(static_cast<uint32_t>(cols / 16)));
    } else {
        size_t blocks = (n + kQThreads - 1) / kQThreads;
        if (blocks > 65536) blocks = 65536;
        dequant_scalar_kernel<MODE><<<dim3(static_cast<unsigned>(blocks)), dim3(kQThreads), 0, stream()>>>(
            static_cast<uint16_t*>(out), static_cast<const int8_t*>(q), static_cast<const float*>(scales), n,
            static_cast<int>(cols));
    }
    NG_CHECK_LAUNCH(name);
    return 0;
}

}  // namespace ng

using namespace ng;

extern "C" int cuda_quantize_per_tensor(void* output, void* scale, const void* input, size_t n) {
    NG_REQUIRE(output && scale && input, "cuda_quantize_per_tensor: null pointer");
    NG_REQUIRE(n > 0, "cuda_quantize_per_tensor: num_elements must be > 0");
    uint32_t* mx = static_cast<uint32_t*>(scale);
    const uint16_t* x = static_cast<const uint16_t*>(input);
    const int vec = aligned16(input) && aligned8(output);
    size_t blocks = (n / 8 + kQThreads - 1) / kQThreads;
    if (blocks < 1) blocks = 1;
    const size_t cap = static_cast<size_t>(device_cu_count()) * 8;
    if (blocks > cap) blocks = cap;
    fill_u32_kernel<<<1, 1, 0, stream()>>>(mx, 1, 0u);
    NG_CHECK_LAUNCH("cuda_quantize_per_tensor");
    tensor_absmax_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(kQThreads), 0, stream()>>>(mx, x, n, vec);
    NG_CHECK_LAUNCH("cuda_quantize_per_tensor");
    tensor_quant_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(kQThreads), 0, stream()>>>(
        static_cast<int8_t*>(output), x, mx, n, vec);
    NG_CHECK_LAUNCH("cuda_quantize_per_tensor");
    tensor_scale_finalize_kernel<<<1, 1, 0, stream()>>>(static_cast<float*>(scale));
    NG_CHECK_LAUNCH("cuda_quantize_per_tensor");
    return 0;
}

extern "C" int cuda_dequantize_per_tensor(void* output, const void* input, const void* scale, size_t n) {
    NG_REQUIRE(output && input && scale, "cuda_dequantize_per_tensor: null pointer");
    NG_REQUIRE(n > 0, "cuda_dequantize_per_tensor: num_elements must be > 0");
    if (n % 16 == 0) return launch_dequant<DQ_TENSOR>("cuda_dequantize_per_tensor", output, input, scale, 1, n);
    return launch_dequant<DQ_TENSOR>("cuda_dequantize_per_tensor", output, input, scale, n, 1);
}

extern "C" int cuda_quantize_weights(void* output, void* scales, const void* input, int K, int N) {
    NG_REQUIRE(output && scales && input, "cuda_quantize_weights: null pointer");
    NG_REQUIRE(K > 0 && N > 0, "cuda_quantize_weights: K=%d N=%d must be > 0", K, N);
    uint32_t* colmax = static_cast<uint32_t*>(scales);
    const uint16_t* x = static_cast<const uint16_t*>(input);
    const int vec = N % 8 == 0 && aligned16(input) && aligned8(output);
    const int cols_per_thread = vec ? 8 : 1;
    const unsigned gx = static_cast<unsigned>((N / cols_per_thread + kQThreads - 1) / kQThreads);
    fill_u32_kernel<<<dim3((N + 255) / 256), dim3(256), 0, stream()>>>(colmax, static_cast<size_t>(N), 0u);
    NG_CHECK_LAUNCH("cuda_quantize_weights");
    const int rows_per_chunk = 64;
    const unsigned chunks = static_cast<unsigned>((K + rows_per_chunk - 1) / rows_per_chunk);
    col_absmax_kernel<<<dim3(gx, chunks), dim3(kQThreads), 0, stream()>>>(colmax, x, K, N, rows_per_chunk, vec);
    NG_CHECK_LAUNCH("cuda_quantize_weights");
    const unsigned gy = static_cast<unsigned>(K < 4096 ? K : 4096);
    col_quant_kernel<<<dim3(gx, gy), dim3(kQThreads), 0, stream()>>>(static_cast<int8_t*>(output), x, colmax, K, N,
                                                                     vec);
    NG_CHECK_LAUNCH("cuda_quantize_weights");
    col_scale_finalize_kernel<<<dim3((N + 255) / 256), dim3(256), 0, stream()>>>(static_cast<float*>(scales), N);
    NG_CHECK_LAUNCH("cuda_quantize_weights");
    return 0;
}

extern "C" int cuda_dequantize_weights(void* output, const void* input, const void* scales, int rows, int cols,
                                       int scale_per_row) {
    NG_REQUIRE(output && input && scales, "cuda_dequantize_weights: null pointer");
    NG_REQUIRE(rows > 0 && cols > 0, "cuda_dequantize_weights: rows=%d cols=%d must be > 0", rows, cols);
    if (scale_per_row)
        return launch_dequant<DQ_ROW>("cuda_dequantize_weights", output, input, scales, rows, cols);
    return launch_dequant<DQ_COL>("cuda_dequantize_weights", output, input, scales, rows, cols);
}
