// ng_common.hpp - shared device/host helpers for the gfx950 kernels.
//
// Element types are the compiler's native _Float16 and __bf16; conversions
// from fp32 round to nearest even (v_cvt_f16_f32, v_cvt_pk_bf16_f32).
// Global memory is moved in 16-byte vectors (8 x 16-bit elements per lane,
// global_load_dwordx4 / global_store_dwordx4).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/stream.h"

namespace ng {

using f16 = _Float16;
using bf16 = __bf16;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Host-side error reporting, mirroring the reference's CUDA_CHECK convention
// (print to stderr, return -1).
// ---------------------------------------------------------------------------
#define NG_REQUIRE(cond, ...)                                    \
    do {                                                         \
        if (!(cond)) {                                           \
            fprintf(stderr, "neurogrid-amd: " __VA_ARGS__);      \
            fputc('\n', stderr);                                 \
            return -1;                                           \
        }                                                        \
    } while (0)

#define NG_CHECK_LAUNCH(name)                                                     \
    do {                                                                          \
        hipError_t ng_err_ = hipGetLastError();                                   \
        if (ng_err_ != hipSuccess) {                                              \
            fprintf(stderr, "neurogrid-amd: %s: launch failed: %s\n", (name),     \
                    hipGetErrorString(ng_err_));                                  \
            return -1;                                                            \
        }                                                                         \
    } while (0)

#define NG_HIP_CHECK(call)                                                        \
    do {                                                                          \
        hipError_t ng_err_ = (call);                                              \
        if (ng_err_ != hipSuccess) {                                              \
            fprintf(stderr, "neurogrid-amd: %s:%d: %s\n", __FILE__, __LINE__,     \
                    hipGetErrorString(ng_err_));                                  \
            return -1;                                                            \
        }                                                                         \
    } while (0)

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

inline hipStream_t stream() { return ng_get_stream(); }

// Number of compute units of the current device (cached per device id).
int device_cu_count();

// ---------------------------------------------------------------------------
// Element conversions.
// ---------------------------------------------------------------------------
template <typename T> __device__ __forceinline__ float to_f32(uint16_t bits);
template <> __device__ __forceinline__ float to_f32<f16>(uint16_t bits) {
    return static_cast<float>(__builtin_bit_cast(f16, bits));
}
template <> __device__ __forceinline__ float to_f32<bf16>(uint16_t bits) {
    return __builtin_bit_cast(float, static_cast<uint32_t>(bits) << 16);
}

template <typename T> __device__ __forceinline__ uint16_t from_f32(float v);
template <> __device__ __forceinline__ uint16_t from_f32<f16>(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<f16>(v));
}
template <> __device__ __forceinline__ uint16_t from_f32<bf16>(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<bf16>(v));
}

// Unpack / pack 8 16-bit elements held in a 16-byte vector.
template <typename T>
__device__ __forceinline__ void unpack8(const u32x4 v, float (&f)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = to_f32<T>(static_cast<uint16_t>(v[i] & 0xffffu));
        f[2 * i + 1] = to_f32<T>(static_cast<uint16_t>(v[i] >> 16));
    }
}

template <typename T>
__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = static_cast<uint32_t>(from_f32<T>(f[2 * i])) |
               (static_cast<uint32_t>(from_f32<T>(f[2 * i + 1])) << 16);
    }
    return v;
}

__device__ __forceinline__ uint16_t lane16(const u32x4 v, int i) {
    return static_cast<uint16_t>((v[i >> 1] >> ((i & 1) * 16)) & 0xffffu);
}

// ---------------------------------------------------------------------------
// 16-byte global memory access. Streaming variants mark the access
// non-temporal so single-use data does not displace reused lines.
// ---------------------------------------------------------------------------
__device__ __forceinline__ u32x4 ld16(const void* p) {
    return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void st16(void* p, u32x4 v) {
    *reinterpret_cast<u32x4*>(p) = v;
}
__device__ __forceinline__ u32x4 ld16_stream(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16_stream(void* p, u32x4 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// ---------------------------------------------------------------------------
// Wave64 reductions (cross-lane butterflies). Every lane ends with the same
// bit pattern: at each level both partners add the same two operands.
// ---------------------------------------------------------------------------
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        uint32_t o = __shfl_xor(v, off, kWave);
        v = v > o ? v : o;
    }
    return v;
}

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ int wave_or(int v) {
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) v |= __shfl_xor(v, off, kWave);
    return v;
}

// ---------------------------------------------------------------------------
// Unsigned 32-bit division by a run-time constant (Granlund-Montgomery
// round-up multiplier): with l = ceil(log2 d) and
// m = floor(2^32 (2^l - d) / d) + 1, n / d = (umulhi(n, m) + n) >> l for
// every 32-bit n and 1 <= d < 2^31.
// ---------------------------------------------------------------------------
struct FastDiv {
    uint32_t d, m, s;
};

inline FastDiv make_fastdiv(uint32_t d) {
    FastDiv f{d, 0, 0};
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    f.m = static_cast<uint32_t>(((1ull << 32) * ((1ull << l) - d)) / d + 1);
    f.s = l;
    return f;
}

__host__ __device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
    uint32_t t = static_cast<uint32_t>((static_cast<uint64_t>(n) * f.m) >> 32);
    return static_cast<uint32_t>((static_cast<uint64_t>(t) + n) >> f.s);
}

}  // namespace ng
