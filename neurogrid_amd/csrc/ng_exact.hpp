// ng_exact.hpp - order-independent sum of squares for the RMSNorm family.
//
// The row statistic is defined as ss = RN_f32(exact sum of v_i^2), the exact
// real sum rounded once to fp32 with ties to even. Its value therefore does
// not depend on how a row is split over lanes and waves, which is what lets
// the GPU result match a sequential CPU oracle bit for bit.
//
// Fast path: every v_i is an fp32 value with at most 24 significant bits, so
// v_i^2 is exact in fp64 and an fp64 sum of n non-negative exact terms, in
// any association order, has relative error below (n-1) 2^-53 (1 + 2^-40).
// With k = ceil(log2 n) the interval S (1 +- 2^(k-51)) therefore contains the
// exact sum; when both of its ends round to the same fp32 value, so does the
// exact sum, and that value is RN_f32(S).
//
// Slow path (taken when an interval end sits on the other side of an fp32
// rounding boundary, about 2^(k-27) of rows): each v_i that lies on the
// 2^-24 grid with |v_i| < 2^20 -- every value derived from fp16 inputs --
// contributes v_i^2 as an exact 128-bit integer in units of 2^-48; the
// integer total is rounded to fp32 exactly.
#pragma once

#include "ng_common.hpp"

namespace ng {

typedef unsigned __int128 u128;

// v^2 in units of 2^-48. Returns false when v is off the 2^-24 grid, has
// |v| >= 2^20, or is not finite (the row then keeps the fast-path value).
__device__ __forceinline__ bool sq_units(float v, u128& out) {
    uint32_t b = __builtin_bit_cast(uint32_t, v) & 0x7fffffffu;
    out = 0;
    if (b == 0) return true;
    uint32_t E = b >> 23;
    if (E == 0 || E >= 147) return false;  // fp32 subnormal, |v| >= 2^20, inf or nan
    uint32_t M = (b & 0x7fffffu) | 0x800000u;
    int tz = __builtin_ctz(M);
    M >>= tz;
    int e = static_cast<int>(E) - 150 + tz;  // v = M * 2^e, M odd
    if (e < -24) return false;
    int sh = 2 * e + 48;                     // 0 <= sh, M^2 2^sh < 2^88
    out = static_cast<u128>(static_cast<uint64_t>(M) * M) << sh;
    return true;
}

// Round a non-negative integer S (units of 2^-48, S < 2^120) to fp32, ties to even.
__device__ __forceinline__ float units_to_f32(u128 S) {
    if (S == 0) return 0.0f;
    uint64_t hi = static_cast<uint64_t>(S >> 64);
    uint64_t lo = static_cast<uint64_t>(S);
    int p = hi ? 127 - __builtin_clzll(hi) : 63 - __builtin_clzll(lo);
    if (p <= 23) return __builtin_ldexpf(static_cast<float>(static_cast<uint32_t>(lo)), -48);
    int sh = p - 23;
    u128 m = S >> sh;
    u128 rem = S - (m << sh);
    u128 half = static_cast<u128>(1) << (sh - 1);
    uint32_t mant = static_cast<uint32_t>(m);
    if (rem > half || (rem == half && (mant & 1u))) ++mant;
    if (mant == (1u << 24)) {
        mant >>= 1;
        ++sh;
    }
    return __builtin_ldexpf(static_cast<float>(mant), sh - 48);
}

// Fast-path resolution of an fp64 sum S of n exact squares (see header).
__device__ __forceinline__ bool ss_fast_resolve(double S, int n, float& ss) {
    ss = static_cast<float>(S);
    if (!__builtin_isfinite(S)) return true;
    int nn = n < 2 ? 2 : n;
    int k = 32 - __builtin_clz(static_cast<uint32_t>(nn - 1));
    double d = __builtin_ldexp(S, k - 51);
    return static_cast<float>(S - d) == static_cast<float>(S + d);
}

__device__ __forceinline__ u128 shfl_xor_u128(u128 v, int off) {
    uint64_t lo = static_cast<uint64_t>(v), hi = static_cast<uint64_t>(v >> 64);
    lo = __shfl_xor(lo, off, kWave);
    hi = __shfl_xor(hi, off, kWave);
    return (static_cast<u128>(hi) << 64) | lo;
}

__device__ __forceinline__ u128 wave_sum_u128(u128 v) {
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) v += shfl_xor_u128(v, off);
    return v;
}

}  // namespace ng
