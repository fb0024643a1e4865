// ng_exact.hpp - order-independent sum of squares for the RMSNorm family.
//
// The row statistic is defined as ss = RN_f32(exact sum of v_i^2), the exact
// real sum rounded once to fp32 with ties to even. Its value therefore does
// not depend on how a row is split over lanes and waves, which is what lets
// the GPU result match a sequential CPU oracle bit for bit.
//
// Fast path. Every v_i is an fp32 value with at most 24 significant bits, so
// v_i^2 is exact in fp64. The squares are summed in fp64 (per-lane
// accumulators, then across lanes and waves). A sum of nonnegative terms
// computed by a summation tree in which no term passes through more than h
// rounded additions differs from the exact sum by at most h u / (1 - h u) of
// it, u = 2^-53 (Higham, Accuracy and Stability of Numerical Algorithms,
// 4.2); callers pass m > h. Where the lanes' partial sums are combined with
// error-free transformations (two_sum), h is that of one lane accumulator.
// With k = ceil(log2 m) + 1, the interval S (1 +- 2^(k-53)) contains the
// exact sum; when both of its ends round to the same fp32 value, that value
// is RN_f32(exact sum). Otherwise (a fraction of about 2^(k-29) of rows: the
// interval is 2^(k-52) S wide, fp32 values are about 2^-23 S apart; 2^-23
// for a row of 4096 held by one wave) the slow path runs.
//
// Slow path. A value v on the 2^-24 grid with |v| < 2^17 (every value derived
// from fp16 inputs) has v^2 = t 2^16 + u 2^-16 + w 2^-48 with integers
// t < 2^18, u < 2^32, w < 2^32, obtained exactly with two fp64 truncations.
// Summed over up to 65536 values each limb stays an integer below 2^53, so
// three fp64 accumulators hold the sum exactly in any order; the limbs are
// then joined into a 128-bit integer (units of 2^-48) and rounded once.
// Rows holding a value off that grid (possible for bf16) keep the fast-path
// value.
#pragma once

#include "ng_common.hpp"

namespace ng {

typedef unsigned __int128 u128;

// ---------------------------------------------------------------- fast path
struct DD {
    double hi, lo;
};

// Error-free a + b. The sums here are of squares, so the only non-finite
// sums come from an inf or NaN in a row: then the error term is 0 and the sum
// itself carries the inf or NaN (the error formula would give inf - inf =
// NaN, turning a row's inf sum of squares into NaN).
__device__ __forceinline__ DD two_sum(double a, double b) {
    const double s = a + b;
    const double bp = s - a;
    const double e = (a - (s - bp)) + (b - bp);
    return {s, __builtin_isfinite(s) ? e : 0.0};
}

// (a.hi + a.lo) + (b.hi + b.lo), renormalised so that |lo| <= ulp(hi) / 2;
// a non-finite hi has lo = 0, as in two_sum.
__device__ __forceinline__ DD dd_add(DD a, DD b) {
    DD s = two_sum(a.hi, b.hi);
    const double lo = s.lo + (a.lo + b.lo);
    const double hi = s.hi + lo;
    return {hi, __builtin_isfinite(hi) ? lo - (hi - s.hi) : 0.0};
}

template <int CTRL>
__device__ __forceinline__ DD dpp_dd(DD v) {
    return {dpp_f64<CTRL>(v.hi), dpp_f64<CTRL>(v.lo)};
}

__device__ __forceinline__ DD readlane_dd(DD v, int lane) {
    return {readlane_f64(v.hi, lane), readlane_f64(v.lo, lane)};
}

// Wave sum with error-free combination; the result is wave-uniform.
__device__ __forceinline__ DD wave_sum_dd(DD v) {
    v = dd_add(v, dpp_dd<kDppQuadSwap1>(v));
    v = dd_add(v, dpp_dd<kDppQuadSwap2>(v));
    v = dd_add(v, dpp_dd<kDppRowHalfMirror>(v));
    v = dd_add(v, dpp_dd<kDppRowMirror>(v));
    return dd_add(dd_add(readlane_dd(v, 0), readlane_dd(v, 16)), dd_add(readlane_dd(v, 32), readlane_dd(v, 48)));
}

// Resolve the fp64 sum S of nonnegative terms (tree height below m, so the
// error is below (m-1) 2^-53 S up to a factor 1 + 2^-40) to RN_f32(exact),
// or report that the slow path is needed.
__device__ __forceinline__ bool ss_fast_resolve(double S, int m, float& ss) {
    ss = static_cast<float>(S);
    if (!__builtin_isfinite(S)) return true;
    const int mm = m < 2 ? 2 : m;
    const int k = 32 - __builtin_clz(static_cast<uint32_t>(mm - 1)) + 1;
    const double d = __builtin_ldexp(S, k - 53);
    return static_cast<float>(S - d) == static_cast<float>(S + d);
}

// ---------------------------------------------------------------- slow path
struct Limbs {
    double t, u, w;  // integer-valued: units of 2^16, 2^-16, 2^-48
    int bad;         // a value off the 2^-24 grid or with |v| >= 2^17
};

__device__ __forceinline__ void limbs_add(Limbs& L, float v) {
    const double d = static_cast<double>(v);
    const double g = d * 0x1p24;
    if (!(__builtin_fabs(d) < 0x1p17) || g != __builtin_trunc(g)) {
        L.bad = 1;
        return;
    }
    const double sq = d * d;                                  // exact, < 2^34
    const double t = __builtin_trunc(sq * 0x1p-16);           // < 2^18
    const double r1 = __builtin_fma(t, -0x1p16, sq);          // exact, in [0, 2^16)
    const double u = __builtin_trunc(r1 * 0x1p16);            // < 2^32
    const double r2 = __builtin_fma(u, -0x1p-16, r1);         // exact, in [0, 2^-16)
    L.t += t;
    L.u += u;
    L.w += r2 * 0x1p48;                                       // < 2^32
}

// Round a non-negative integer S (units of 2^-48, S < 2^120) to fp32, ties to even.
__device__ __forceinline__ float units_to_f32(u128 S) {
    if (S == 0) return 0.0f;
    const uint64_t hi = static_cast<uint64_t>(S >> 64);
    const uint64_t lo = static_cast<uint64_t>(S);
    const int p = hi ? 127 - __builtin_clzll(hi) : 63 - __builtin_clzll(lo);
    if (p <= 23) return __builtin_ldexpf(static_cast<float>(static_cast<uint32_t>(lo)), -48);
    int sh = p - 23;
    const u128 m = S >> sh;
    const u128 rem = S - (m << sh);
    const u128 half = static_cast<u128>(1) << (sh - 1);
    uint32_t mant = static_cast<uint32_t>(m);
    if (rem > half || (rem == half && (mant & 1u))) ++mant;
    if (mant == (1u << 24)) {
        mant >>= 1;
        ++sh;
    }
    return __builtin_ldexpf(static_cast<float>(mant), sh - 48);
}

// Exact total of the three limb sums, rounded to fp32.
__device__ __forceinline__ float limbs_to_f32(double t, double u, double w) {
    const u128 S = (static_cast<u128>(static_cast<uint64_t>(t)) << 64) +
                   (static_cast<u128>(static_cast<uint64_t>(u)) << 32) + static_cast<u128>(static_cast<uint64_t>(w));
    return units_to_f32(S);
}

}  // namespace ng
