// elementwise.hip - streaming element-wise kernels: SwiGLU (silu * up), SiLU,
// add, mul, scale, and the fp16/bf16/fp32 converters.
//
// Semantics, in fp32 with one final round-to-nearest-even to the element type
// (reference: gpu/cuda/kernels.cu:126-188, 269-359, 653-664; bf16_utils.cu:122-321):
//   add  c = RN(a + b)           mul  c = RN(a * b)        scale y = RN(x * s)
//   silu y = RN(x * sig(x))      silu_mul out = RN((g * sig(g)) * u)
//   sig(x) = 1 / (1 + exp(-x))
// add, mul and scale are exact-rounded; exp and the reciprocal in sig use the
// hardware v_exp_f32 / v_rcp_f32 (a few fp32 ulp, far below half an ulp of
// the 16-bit result).
//
// Layout: each thread moves U 16-byte vectors per operand (8 elements each),
// lane-contiguous so a wave covers 1 KiB per operand per vector; loads and
// stores are non-temporal because every byte is used exactly once.
#include "ng_common.hpp"

namespace ng {

enum EwOp : int { EW_ADD = 0, EW_MUL = 1, EW_SILU = 2, EW_SILU_MUL = 3, EW_SCALE = 4 };

template <int OP>
__device__ __forceinline__ float ew_apply(float a, float b, float s) {
    if (OP == EW_ADD) return a + b;
    if (OP == EW_MUL) return a * b;
    if (OP == EW_SILU) return a * sigmoid_fast(a);
    if (OP == EW_SILU_MUL) return swiglu_f32(a, b);
    return a * s;  // EW_SCALE
}

template <int OP>
struct EwArity {
    static constexpr bool binary = (OP == EW_ADD || OP == EW_MUL || OP == EW_SILU_MUL);
};

// One wave per workgroup: measured on MI355X, 64-thread workgroups are 6-7%
// faster than 256-thread ones for the streaming kernels here (SwiGLU on
// [4096, 14336]: 53.4 vs 57.5 us; residual add on [4096, 4096]: 16.4 vs
// 17.4 us), and 128 threads fall in between.
constexpr int kEwThreads = 64;
// One 16-byte vector per operand per thread: measured on MI355X, deeper
// per-thread unrolling (2 or 4 vectors) is slower at every size from 0.5 MB
// to 350 MB, and at decode sizes it leaves most CUs idle.
constexpr int kEwUnroll = 1;

template <typename T, int OP, int U>
__global__ __launch_bounds__(kEwThreads) void ew_vec_kernel(void* out, const void* a, const void* b,
                                                            float s, size_t nvec) {
    const size_t base = static_cast<size_t>(blockIdx.x) * (kEwThreads * U) + threadIdx.x;
    const uint16_t* A = static_cast<const uint16_t*>(a);
    const uint16_t* B = static_cast<const uint16_t*>(b);
    uint16_t* O = static_cast<uint16_t*>(out);
    u32x4 va[U], vb[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
        const size_t i = base + static_cast<size_t>(k) * kEwThreads;
        if (i < nvec) {
            va[k] = ld16_stream(A + i * 8);
            if (EwArity<OP>::binary) vb[k] = ld16_stream(B + i * 8);
        }
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
        const size_t i = base + static_cast<size_t>(k) * kEwThreads;
        if (i < nvec) {
            float fa[8], fb[8], fo[8];
            unpack8<T>(va[k], fa);
            if (EwArity<OP>::binary) unpack8<T>(vb[k], fb);
#pragma unroll
            for (int e = 0; e < 8; ++e) fo[e] = ew_apply<OP>(fa[e], EwArity<OP>::binary ? fb[e] : 0.0f, s);
            st16_stream(O + i * 8, pack8<T>(fo));
        }
    }
}

// Any length and alignment: one element per thread per step.
template <typename T, int OP>
__global__ __launch_bounds__(kEwThreads) void ew_scalar_kernel(void* out, const void* a, const void* b,
                                                               float s, size_t begin, size_t n) {
    const uint16_t* A = static_cast<const uint16_t*>(a);
    const uint16_t* B = static_cast<const uint16_t*>(b);
    uint16_t* O = static_cast<uint16_t*>(out);
    const size_t stride = static_cast<size_t>(gridDim.x) * kEwThreads;
    for (size_t i = begin + static_cast<size_t>(blockIdx.x) * kEwThreads + threadIdx.x; i < n; i += stride) {
        const float fa = to_f32<T>(A[i]);
        const float fb = EwArity<OP>::binary ? to_f32<T>(B[i]) : 0.0f;
        O[i] = from_f32<T>(ew_apply<OP>(fa, fb, s));
    }
}

template <typename T, int OP>
static int launch_ew(const char* name, void* out, const void* a, const void* b, float s, size_t n) {
    NG_REQUIRE(out && a && (!EwArity<OP>::binary || b), "%s: null pointer", name);
    NG_REQUIRE(n > 0, "%s: num_elements must be > 0", name);
    const bool vec = aligned16(out) && aligned16(a) && (!EwArity<OP>::binary || aligned16(b));
    size_t done = 0;
    if (vec) {
        const size_t nvec = n / 8;
        if (nvec > 0) {
            const size_t per_block = static_cast<size_t>(kEwThreads) * kEwUnroll;
            const size_t blocks = (nvec + per_block - 1) / per_block;
            ew_vec_kernel<T, OP, kEwUnroll><<<dim3(static_cast<unsigned>(blocks)), dim3(kEwThreads), 0, stream()>>>(
                out, a, b, s, nvec);
            NG_CHECK_LAUNCH(name);
        }
        done = nvec * 8;
    }
    if (done < n) {
        const size_t rem = n - done;
        size_t blocks = (rem + kEwThreads - 1) / kEwThreads;
        if (blocks > 65536) blocks = 65536;
        ew_scalar_kernel<T, OP><<<dim3(static_cast<unsigned>(blocks)), dim3(kEwThreads), 0, stream()>>>(
            out, a, b, s, done, n);
        NG_CHECK_LAUNCH(name);
    }
    return 0;
}

// ---------------------------------------------------------------------------
// Converters. 16-bit side in 16-byte vectors of 8; fp32 side in two vectors.
// ---------------------------------------------------------------------------
enum CvtKind : int { CVT_BF16_TO_F32 = 0, CVT_F32_TO_BF16 = 1, CVT_F16_TO_BF16 = 2, CVT_BF16_TO_F16 = 3,
                     CVT_F32_TO_F16 = 4, CVT_F16_TO_F32 = 5 };

template <int K>
__device__ __forceinline__ void cvt_load8(const void* in, size_t e0, float (&f)[8]) {
    if (K == CVT_F32_TO_BF16 || K == CVT_F32_TO_F16) {
        const u32x4 v0 = ld16_stream(static_cast<const float*>(in) + e0);
        const u32x4 v1 = ld16_stream(static_cast<const float*>(in) + e0 + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[i] = as_float(v0[i]);
            f[4 + i] = as_float(v1[i]);
        }
    } else {
        const u32x4 v = ld16_stream(static_cast<const uint16_t*>(in) + e0);
        if (K == CVT_F16_TO_BF16 || K == CVT_F16_TO_F32) unpack8<f16>(v, f);
        else unpack8<bf16>(v, f);
    }
}

template <int K>
__device__ __forceinline__ void cvt_store8(void* out, size_t e0, const float (&f)[8]) {
    if (K == CVT_BF16_TO_F32 || K == CVT_F16_TO_F32) {
        u32x4 v0, v1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v0[i] = __builtin_bit_cast(uint32_t, f[i]);
            v1[i] = __builtin_bit_cast(uint32_t, f[4 + i]);
        }
        st16_stream(static_cast<float*>(out) + e0, v0);
        st16_stream(static_cast<float*>(out) + e0 + 4, v1);
    } else if (K == CVT_BF16_TO_F16 || K == CVT_F32_TO_F16) {
        st16_stream(static_cast<uint16_t*>(out) + e0, pack8<f16>(f));
    } else {
        st16_stream(static_cast<uint16_t*>(out) + e0, pack8<bf16>(f));
    }
}

template <int K>
__device__ __forceinline__ float cvt_load1(const void* in, size_t i) {
    if (K == CVT_F32_TO_BF16 || K == CVT_F32_TO_F16) return static_cast<const float*>(in)[i];
    const uint16_t b = static_cast<const uint16_t*>(in)[i];
    return (K == CVT_F16_TO_BF16 || K == CVT_F16_TO_F32) ? to_f32<f16>(b) : to_f32<bf16>(b);
}

template <int K>
__device__ __forceinline__ void cvt_store1(void* out, size_t i, float v) {
    if (K == CVT_BF16_TO_F32 || K == CVT_F16_TO_F32) static_cast<float*>(out)[i] = v;
    else if (K == CVT_BF16_TO_F16 || K == CVT_F32_TO_F16) static_cast<uint16_t*>(out)[i] = from_f32<f16>(v);
    else static_cast<uint16_t*>(out)[i] = from_f32<bf16>(v);
}

// One 8-element vector per thread, one-wave workgroups, as the element-wise
// kernels (timed the same as a grid-stride loop over 64 workgroups per CU).
template <int K>
__global__ __launch_bounds__(kEwThreads) void cvt_vec_kernel(void* out, const void* in, size_t nvec) {
    const size_t i = static_cast<size_t>(blockIdx.x) * kEwThreads + threadIdx.x;
    if (i >= nvec) return;
    float f[8];
    cvt_load8<K>(in, i * 8, f);
    cvt_store8<K>(out, i * 8, f);
}

// Elements [start, n) one per thread per step (the tail, or unaligned buffers).
template <int K>
__global__ __launch_bounds__(kEwThreads) void cvt_scalar_kernel(void* out, const void* in, size_t start, size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * kEwThreads;
    for (size_t i = start + static_cast<size_t>(blockIdx.x) * kEwThreads + threadIdx.x; i < n; i += stride)
        cvt_store1<K>(out, i, cvt_load1<K>(in, i));
}

// Grid for one thread per unit, or for a grid-stride loop over a tail.
static unsigned ew_blocks(size_t units, size_t cap) {
    size_t blocks = (units + kEwThreads - 1) / kEwThreads;
    if (blocks < 1) blocks = 1;
    if (blocks > cap) blocks = cap;
    return static_cast<unsigned>(blocks);
}

template <int K>
static int launch_cvt(const char* name, void* out, const void* in, size_t n) {
    NG_REQUIRE(out && in, "%s: null pointer", name);
    NG_REQUIRE(n > 0, "%s: num_elements must be > 0", name);
    size_t done = 0;
    if (aligned16(out) && aligned16(in)) {
        const size_t nvec = n / 8;
        NG_REQUIRE(nvec / kEwThreads < 0xffffffffull, "%s: tensor too large", name);
        if (nvec > 0) {
            cvt_vec_kernel<K><<<dim3(ew_blocks(nvec, ~0u)), dim3(kEwThreads), 0, stream()>>>(out, in, nvec);
            NG_CHECK_LAUNCH(name);
        }
        done = nvec * 8;
    }
    if (done < n) {
        cvt_scalar_kernel<K><<<dim3(ew_blocks(n - done, 65536)), dim3(kEwThreads), 0, stream()>>>(out, in, done, n);
        NG_CHECK_LAUNCH(name);
    }
    return 0;
}

// bf16 -> fp16 as the model loader converts weights on the host
// (pkg/model/loader.go:23-85): through fp32, then the fp16 mantissa is
// truncated, fp16-subnormal results truncate toward zero, magnitudes from
// 2^16 up become infinity, NaN becomes 0x7E00 with its sign, and values below
// 2^-24 become a signed zero. bf16's 7 mantissa bits fit in fp16's 10, so in
// fp16's normal range the value is exact; the rest is integer bit work.
__device__ __forceinline__ uint32_t bf16_to_f16_trunc(uint32_t b) {
    const uint32_t sign = (b & 0x8000u);
    const int e8 = static_cast<int>((b >> 7) & 0xffu);
    const uint32_t m7 = b & 0x7fu;
    const int e16 = e8 - 112;  // fp16 biased exponent
    uint32_t mag;
    if (e8 == 0xff) mag = m7 == 0 ? 0x7c00u : 0x7e00u;
    else if (e16 >= 31) mag = 0x7c00u;
    else if (e16 >= 1) mag = (static_cast<uint32_t>(e16) << 10) | (m7 << 3);
    else if (e16 >= -10) mag = ((m7 | 0x80u) << 16) >> (14 - e16);
    else mag = 0u;
    return sign | mag;
}

__global__ __launch_bounds__(kEwThreads) void bf16_to_f16_trunc_vec_kernel(uint16_t* out, const uint16_t* in,
                                                                           size_t nvec) {
    const size_t i = static_cast<size_t>(blockIdx.x) * kEwThreads + threadIdx.x;
    if (i >= nvec) return;
    u32x4 v = ld16_stream(in + i * 8);
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = bf16_to_f16_trunc(v[j] & 0xffffu) | (bf16_to_f16_trunc(v[j] >> 16) << 16);
    st16_stream(out + i * 8, v);
}

__global__ __launch_bounds__(kEwThreads) void bf16_to_f16_trunc_scalar_kernel(uint16_t* out, const uint16_t* in,
                                                                              size_t start, size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * kEwThreads;
    for (size_t i = start + static_cast<size_t>(blockIdx.x) * kEwThreads + threadIdx.x; i < n; i += stride)
        out[i] = static_cast<uint16_t>(bf16_to_f16_trunc(in[i]));
}

}  // namespace ng

using namespace ng;

extern "C" int cuda_add(void* c, const void* a, const void* b, size_t n) {
    return launch_ew<f16, EW_ADD>("cuda_add", c, a, b, 0.0f, n);
}
extern "C" int cuda_mul(void* c, const void* a, const void* b, size_t n) {
    return launch_ew<f16, EW_MUL>("cuda_mul", c, a, b, 0.0f, n);
}
extern "C" int cuda_silu(void* output, const void* input, size_t n) {
    return launch_ew<f16, EW_SILU>("cuda_silu", output, input, nullptr, 0.0f, n);
}
extern "C" int cuda_silu_mul(void* output, const void* gate, const void* up, size_t n) {
    return launch_ew<f16, EW_SILU_MUL>("cuda_silu_mul", output, gate, up, 0.0f, n);
}
extern "C" int cuda_scale(void* output, const void* input, float scale, size_t n) {
    return launch_ew<f16, EW_SCALE>("cuda_scale", output, input, nullptr, scale, n);
}
extern "C" int cuda_bf16_add(void* c, const void* a, const void* b, size_t n) {
    return launch_ew<bf16, EW_ADD>("cuda_bf16_add", c, a, b, 0.0f, n);
}
extern "C" int cuda_bf16_mul(void* c, const void* a, const void* b, size_t n) {
    return launch_ew<bf16, EW_MUL>("cuda_bf16_mul", c, a, b, 0.0f, n);
}
extern "C" int cuda_bf16_silu(void* output, const void* input, size_t n) {
    return launch_ew<bf16, EW_SILU>("cuda_bf16_silu", output, input, nullptr, 0.0f, n);
}
extern "C" int ng_bf16_silu_mul(void* output, const void* gate, const void* up, size_t n) {
    return launch_ew<bf16, EW_SILU_MUL>("ng_bf16_silu_mul", output, gate, up, 0.0f, n);
}
extern "C" int cuda_bf16_to_fp32(void* output, const void* input, size_t n) {
    return launch_cvt<CVT_BF16_TO_F32>("cuda_bf16_to_fp32", output, input, n);
}
extern "C" int cuda_fp32_to_bf16(void* output, const void* input, size_t n) {
    return launch_cvt<CVT_F32_TO_BF16>("cuda_fp32_to_bf16", output, input, n);
}
extern "C" int cuda_fp16_to_bf16(void* output, const void* input, size_t n) {
    return launch_cvt<CVT_F16_TO_BF16>("cuda_fp16_to_bf16", output, input, n);
}
extern "C" int cuda_bf16_to_fp16(void* output, const void* input, size_t n) {
    return launch_cvt<CVT_BF16_TO_F16>("cuda_bf16_to_fp16", output, input, n);
}
extern "C" int ng_fp32_to_fp16(void* output, const void* input, size_t n) {
    return launch_cvt<CVT_F32_TO_F16>("ng_fp32_to_fp16", output, input, n);
}
extern "C" int ng_fp16_to_fp32(void* output, const void* input, size_t n) {
    return launch_cvt<CVT_F16_TO_F32>("ng_fp16_to_fp32", output, input, n);
}
extern "C" int ng_bf16_to_fp16_truncate(void* output, const void* input, size_t n) {
    NG_REQUIRE(output && input, "ng_bf16_to_fp16_truncate: null pointer");
    NG_REQUIRE(n > 0, "ng_bf16_to_fp16_truncate: num_elements must be > 0");
    auto* o = static_cast<uint16_t*>(output);
    const auto* x = static_cast<const uint16_t*>(input);
    size_t done = 0;
    if (aligned16(output) && aligned16(input)) {
        const size_t nvec = n / 8;
        NG_REQUIRE(nvec / kEwThreads < 0xffffffffull, "ng_bf16_to_fp16_truncate: tensor too large");
        if (nvec > 0) {
            bf16_to_f16_trunc_vec_kernel<<<dim3(ew_blocks(nvec, ~0u)), dim3(kEwThreads), 0, stream()>>>(o, x, nvec);
            NG_CHECK_LAUNCH("ng_bf16_to_fp16_truncate");
        }
        done = nvec * 8;
    }
    if (done < n)
        bf16_to_f16_trunc_scalar_kernel<<<dim3(ew_blocks(n - done, 65536)), dim3(kEwThreads), 0, stream()>>>(
            o, x, done, n);
    NG_CHECK_LAUNCH("ng_bf16_to_fp16_truncate");
    return 0;
}
