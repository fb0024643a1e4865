// ng_common.hpp - shared device/host helpers for the gfx950 kernels.
//
// Element types are the compiler's native _Float16 and __bf16; conversions
// from fp32 round to nearest even (v_cvt_pk_f16_f32, v_cvt_pk_bf16_f32).
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

// RoPE's inverse frequencies 1 / theta^(2 i / D), i < D / 2, as every RoPE
// launch takes them (rope.hip; cached per theta and D).
void fill_inv_freq(float theta, int D, float* dst);

// Frees every buffer, plan and library handle held by the GEMM entry points
// (matmul.hip), on every device. cuda_shutdown calls it before it resets the
// device, which would otherwise leave them pointing at released memory.
__attribute__((visibility("hidden"))) void gemm_release();

// Looks up, with device `dev` current, the device address of the fixed
// partial-sum array of ng_gemm_int8_noalloc (matmul.hip) and keeps it for
// that device. cuda_init calls it; the entry point also does on its first
// call on a device. Returns 0 or -1.
__attribute__((visibility("hidden"))) int gemm_scratch_init(int dev);

// RMSNorm of `rows` rows of H 16-bit elements through the row kernels
// (norm.hip); launches on stream(), returns 0 or -1.
template <typename T>
__attribute__((visibility("hidden"))) int rows_rmsnorm(const char* name, void* output, const void* input,
                                                      const void* weight, int rows, int H, float eps);

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

// Reinterpret a 32-bit lane as fp32. Takes the lane by value: clang's
// __builtin_bit_cast applied directly to an ext_vector element (v[i]) reads
// element 0 instead of element i.
__device__ __forceinline__ float as_float(uint32_t bits) { return __builtin_bit_cast(float, bits); }

// fp32 -> 16-bit, round to nearest even, from a value already rounded to
// fp32. The empty asm makes the fp32 value opaque: without it the backend
// folds "multiply, then convert to f16" into one v_fma_mixlo_f16, which
// rounds once from the exact product and so differs from the fp32-then-f16
// rounding these kernels are specified with (about 1 element in 2^14).
__device__ __forceinline__ float fp32_barrier(float v) {
    __asm__("" : "+v"(v));
    return v;
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

template <typename T> __device__ __forceinline__ uint16_t from_f32(float v);
template <> __device__ __forceinline__ uint16_t from_f32<f16>(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<f16>(fp32_barrier(v)));
}
template <> __device__ __forceinline__ uint16_t from_f32<bf16>(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<bf16>(fp32_barrier(v)));
}

// Two fp32 values -> one dword of two 16-bit values (v_cvt_pk_f16_f32 /
// v_cvt_pk_bf16_f32, round to nearest even), low half first.
template <typename T> __device__ __forceinline__ uint32_t pack2(float a, float b);
template <> __device__ __forceinline__ uint32_t pack2<f16>(float a, float b) {
    const f32x2 v = {fp32_barrier(a), fp32_barrier(b)};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}
template <> __device__ __forceinline__ uint32_t pack2<bf16>(float a, float b) {
    const f32x2 v = {fp32_barrier(a), fp32_barrier(b)};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
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
    for (int i = 0; i < 4; ++i) v[i] = pack2<T>(f[2 * i], f[2 * i + 1]);
    return v;
}

// sig(x) = 1 / (1 + exp(-x)) with the hardware exp2 and reciprocal
// (v_exp_f32 / v_rcp_f32: a few fp32 ulp, far below half an ulp of a 16-bit
// result), and SwiGLU's element silu(g) * u = (g * sig(g)) * u in fp32. The
// element-wise kernels and the GEMV's SwiGLU epilogue share these, so both
// round the same fp32 value.
__device__ __forceinline__ float sigmoid_fast(float x) {
    const float e = __builtin_amdgcn_exp2f(-x * 1.4426950408889634f);
    return __builtin_amdgcn_rcpf(1.0f + e);
}
__device__ __forceinline__ float swiglu_f32(float g, float u) { return (g * sigmoid_fast(g)) * u; }

__device__ __forceinline__ uint16_t lane16(const u32x4 v, int i) {
    return static_cast<uint16_t>((v[i >> 1] >> ((i & 1) * 16)) & 0xffffu);
}

// ---------------------------------------------------------------------------
// Arithmetic on one 16-bit element of a packed dword (HI selects the upper
// half), each rounded once to fp32 exactly as the plain fp32 expression
// would be. For fp16 each is one v_fma_mix_f32, which widens its fp16
// operands exactly inside the instruction, so no separate conversion is
// issued; for bf16 the element is widened with a shift first.
//   el_get  h            el_mul  RN(h * b)        el_add  RN(ha + hb)
//   el_fma  RN(a * b + h)
// el_mul adds -0.0 to the exact product so that a zero product keeps the
// sign an IEEE multiply gives it.
// ---------------------------------------------------------------------------
template <typename T, int HI>
__device__ __forceinline__ float el_get(uint32_t p) {
    return to_f32<T>(static_cast<uint16_t>(HI ? p >> 16 : p & 0xffffu));
}

template <typename T, int HI>
__device__ __forceinline__ float el_mul(uint32_t p, float b) {
    if constexpr (__is_same(T, f16)) {
        float d;
        if (HI)
            __asm__("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(d) : "v"(p), "v"(b), "v"(-0.0f));
        else
            __asm__("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(d) : "v"(p), "v"(b), "v"(-0.0f));
        return d;
    } else {
        return fp32_barrier(el_get<T, HI>(p) * b);
    }
}

template <typename T, int HI>
__device__ __forceinline__ float el_add(uint32_t pa, uint32_t pb) {
    if constexpr (__is_same(T, f16)) {
        float d;
        if (HI)
            __asm__("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,1] op_sel_hi:[1,0,1]" : "=v"(d) : "v"(pa), "v"(pb));
        else
            __asm__("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,1]" : "=v"(d) : "v"(pa), "v"(pb));
        return d;
    } else {
        return fp32_barrier(el_get<T, HI>(pa) + el_get<T, HI>(pb));
    }
}

template <typename T, int HI>
__device__ __forceinline__ float el_fma(float a, float b, uint32_t p) {
    if constexpr (__is_same(T, f16)) {
        float d;
        if (HI)
            __asm__("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,0,1] op_sel_hi:[0,0,1]" : "=v"(d) : "v"(a), "v"(b), "v"(p));
        else
            __asm__("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[0,0,1]" : "=v"(d) : "v"(a), "v"(b), "v"(p));
        return d;
    } else {
        return __builtin_fmaf(a, b, el_get<T, HI>(p));
    }
}

// ---------------------------------------------------------------------------
// int8 absmax code: q = clamp(rint(RN(v / s)), -127, 127) for a row scale
// s = RN(m / 127) > 0 of the row's absmax m, given inv = RN(1 / s) and
// ns = -s. RN(v / s) is obtained without a division: z = RN(v inv) is within
// a few ulp of v / s, the residual r = RN(v - z s) is then exact, and
// z1 = RN(z + r inv) is the correctly rounded quotient (Markstein's correction
// step). Adding 1.5 * 2^23 to z1 rounds it to an integer, ties to even, and
// leaves that integer in the low bits of the sum, so its low byte is the
// two's-complement code. No clamp is needed: |v| <= m gives
// |v / s| <= 127 (1 + 2^-24). The whole sequence is checked exhaustively
// against clamp(rint(v / s)) with IEEE division, for every fp16 m and every
// fp16 v with |v| <= m.
// ---------------------------------------------------------------------------
constexpr float kRoundMagic = 12582912.0f;  // 1.5 * 2^23

template <typename T, int HI>
__device__ __forceinline__ uint32_t qcode_bits(uint32_t p, float inv, float ns) {
    float z1;
    if constexpr (__is_same(T, f16)) {
        const float z = el_mul<T, HI>(p, inv);
        const float r = el_fma<T, HI>(z, ns, p);
        z1 = __builtin_fmaf(r, inv, z);
    } else {
        const float v = el_get<T, HI>(p);
        const float z = v * inv;
        z1 = __builtin_fmaf(__builtin_fmaf(z, ns, v), inv, z);
    }
    return __builtin_bit_cast(uint32_t, fp32_barrier(z1) + kRoundMagic);
}

// Codes of the 8 elements of a 16-byte vector, as two dwords of int8.
template <typename T>
__device__ __forceinline__ u32x2 qcode8(const u32x4 v, float inv, float ns) {
    u32x2 out;
#pragma unroll
    for (int d = 0; d < 2; ++d) {
        const uint32_t b0 = qcode_bits<T, 0>(v[2 * d], inv, ns), b1 = qcode_bits<T, 1>(v[2 * d], inv, ns);
        const uint32_t b2 = qcode_bits<T, 0>(v[2 * d + 1], inv, ns), b3 = qcode_bits<T, 1>(v[2 * d + 1], inv, ns);
        const uint32_t lo = __builtin_amdgcn_perm(b1, b0, 0x0c0c0400u);  // bytes b0.0, b1.0, 0, 0
        const uint32_t hi = __builtin_amdgcn_perm(b3, b2, 0x0c0c0400u);  // bytes b2.0, b3.0, 0, 0
        out[d] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);            // lo.0, lo.1, hi.0, hi.1
    }
    return out;
}

// The reference's clamp of a rounded quotient, fmaxf(-127, fminf(127, q))
// (quantize.cu:92,228,313). fminf returns its other operand when one is NaN,
// so a NaN quotient (a NaN element, or inf / inf) gives +127.
__device__ __forceinline__ int qclamp_ref(float q) { return static_cast<int>(fmaxf(-127.0f, fminf(127.0f, q))); }

// Codes of a row that holds a NaN or whose scale is not finite: the IEEE
// quotient itself, rounded and clamped as the reference does. Finite values
// of a row with an infinite scale get code 0, as v / inf = 0 (the correction
// step above would form 0 * inf = NaN instead); NaN elements, and infinite
// elements of a row with an infinite scale, get +127.
template <typename T>
__device__ __forceinline__ u32x2 qcode8_div(const u32x4 v, float scale) {
    u32x2 out = {0, 0};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int c = qclamp_ref(__builtin_rintf(to_f32<T>(lane16(v, e)) / scale));
        out[e >> 2] |= (static_cast<uint32_t>(c) & 0xffu) << ((e & 3) * 8);
    }
    return out;
}

// Scalar form of the code (for element-wise fallback paths); a non-finite
// element or scale takes the IEEE quotient, like qcode8_div.
__device__ __forceinline__ int qcode_int(float v, float scale, float inv) {
    if (!__builtin_isfinite(scale) || !__builtin_isfinite(v)) return qclamp_ref(__builtin_rintf(v / scale));
    const float z = v * inv;
    const float z1 = __builtin_fmaf(__builtin_fmaf(z, -scale, v), inv, z);
    return static_cast<int8_t>(__builtin_bit_cast(uint32_t, fp32_barrier(z1) + kRoundMagic) & 0xffu);
}

// Magnitude pattern of +inf in the 16-bit format; larger patterns are NaNs.
template <typename T> inline constexpr uint32_t kInfBits = 0x7c00u;
template <> inline constexpr uint32_t kInfBits<bf16> = 0x7f80u;

// Largest |value| of the 8 elements of a 16-byte vector, as the 15-bit
// magnitude pattern (for non-NaN values |a| < |b| iff the patterns compare
// so). A NaN pattern ranks above +inf: a result above kInfBits<T> says the
// vectors held a NaN, and absmax_bits8_nonan then gives the maximum the
// reference's fmaxf reduction takes, which skips NaNs (quantize.cu:24-50).
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t absmax_bits8(const u32x4 v, uint32_t m) {
    u16x2 a = __builtin_bit_cast(u16x2, v[0] & 0x7fff7fffu);
    a = __builtin_elementwise_max(a, __builtin_bit_cast(u16x2, v[1] & 0x7fff7fffu));
    a = __builtin_elementwise_max(a, __builtin_bit_cast(u16x2, v[2] & 0x7fff7fffu));
    a = __builtin_elementwise_max(a, __builtin_bit_cast(u16x2, v[3] & 0x7fff7fffu));
    const uint32_t r = a[0] > a[1] ? a[0] : a[1];
    return r > m ? r : m;
}

template <typename T>
__device__ __forceinline__ uint32_t absmax_bits8_nonan(const u32x4 v, uint32_t m) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t b = lane16(v, e) & 0x7fffu;
        if (b <= kInfBits<T> && b > m) m = b;
    }
    return m;
}

// Magnitude pattern of one element for an absmax that skips NaNs (0 for a NaN).
template <typename T>
__device__ __forceinline__ uint32_t absbits_nonan(uint16_t bits) {
    const uint32_t b = bits & 0x7fffu;
    return b > kInfBits<T> ? 0u : b;
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
// Device-scope store (sc1) of 16 bytes at byte offset `off` of the buffer
// `r`. For small tensors updated in place (RoPE up to 8 MiB) it measured
// faster than the non-temporal store on MI355X; for large ones, and for the
// kernels that write a separate output, slower. Written with the buffer-store
// builtin (cache-policy operand 16 = sc1 on gfx950), not inline asm, so that
// the compiler sees the store and keeps the wait states a VALU write to its
// data registers needs after it.
constexpr int kCachePolicySC1 = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(base, 0, static_cast<int>(bytes), 0x00020000);
}
__device__ __forceinline__ void st16_device(__amdgpu_buffer_rsrc_t r, uint32_t off, u32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kCachePolicySC1);
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

// DPP variants: four in-row butterflies (quad_perm 1032, quad_perm 2301,
// row_half_mirror, row_mirror) leave every lane of a 16-lane row with the
// row total; the four row totals are read with v_readlane and combined in a
// fixed order, so the result is wave-uniform (scalar) and identical in every
// lane. No LDS round trip, unlike the __shfl_xor (ds_bpermute) versions.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xf, 0xf, false));
}

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = dpp_u32<CTRL>(static_cast<uint32_t>(b));
    const uint64_t hi = dpp_u32<CTRL>(static_cast<uint32_t>(b >> 32));
    return __builtin_bit_cast(double, (hi << 32) | lo);
}

__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, int lane) {
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), lane));
}

__device__ __forceinline__ double readlane_f64(double v, int lane) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = readlane_u32(static_cast<uint32_t>(b), lane);
    const uint64_t hi = readlane_u32(static_cast<uint32_t>(b >> 32), lane);
    return __builtin_bit_cast(double, (hi << 32) | lo);
}

constexpr int kDppQuadSwap1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

__device__ __forceinline__ double wave_sum_f64_dpp(double v) {
    v += dpp_f64<kDppQuadSwap1>(v);
    v += dpp_f64<kDppQuadSwap2>(v);
    v += dpp_f64<kDppRowHalfMirror>(v);
    v += dpp_f64<kDppRowMirror>(v);
    return (readlane_f64(v, 0) + readlane_f64(v, 16)) + (readlane_f64(v, 32) + readlane_f64(v, 48));
}

__device__ __forceinline__ uint32_t umax32(uint32_t a, uint32_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint32_t wave_max_u32_dpp(uint32_t v) {
    v = umax32(v, dpp_u32<kDppQuadSwap1>(v));
    v = umax32(v, dpp_u32<kDppQuadSwap2>(v));
    v = umax32(v, dpp_u32<kDppRowHalfMirror>(v));
    v = umax32(v, dpp_u32<kDppRowMirror>(v));
    return umax32(umax32(readlane_u32(v, 0), readlane_u32(v, 16)), umax32(readlane_u32(v, 32), readlane_u32(v, 48)));
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
