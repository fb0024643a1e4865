/* Exhaustive check of the division-free int8 codes the GPU kernels compute
 * (qcode8 and qcode_int in neurogrid_amd/csrc/ng_common.hpp), against the
 * reference's rule q = clamp(rint(v / s), -127, 127) with the IEEE quotient
 * (gpu/cuda/quantize.cu:292-313, half-to-even rounding), for every positive
 * finite fp16 row absmax m, s = RN(m / 127), and every finite fp16 v with
 * |v| <= m (the values a row with that absmax holds):
 *   z = RN(v inv), r = RN(v - z s), z1 = RN(z + r inv) (Markstein's
 *   correction step), code = low byte of RN(z1 + 1.5 2^23).
 * Also counted, for comparison: the plain product z (without the correction)
 * and a two-product bracket, t_lo = RN(v inv_lo + 1.5 2^23),
 * t_hi = RN(v inv_hi + 1.5 2^23) with inv_lo / inv_hi = RN(inv (1 -/+ 2^-22)),
 * which is right wherever t_lo == t_hi but leaves undecided every v / s near a
 * half-integer, among them v = m / 2 (q = 63.5), common in fp16 rows.
 *
 * inv = RN(1 / s). Every operation is one IEEE fp32 rounding (fmaf is fused,
 * build with -ffp-contract=off), as on the GPU (v_fma_mix_f32 widens the fp16
 * operand exactly and rounds once). Prints the counts; exits 1 on any wrong
 * code. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float h2f(uint16_t h) {
    int e = (h >> 10) & 0x1f, m = h & 0x3ff;
    float v = e == 0 ? ldexpf((float)m, -24) : ldexpf((float)(m | 0x400), e - 25);
    return (h & 0x8000) ? -v : v;
}

static int low_code(float t) {
    uint32_t b;
    memcpy(&b, &t, 4);
    return (int)(int8_t)(b & 0xffu);
}

int main(void) {
    const float M = 12582912.0f; /* 1.5 * 2^23 */
    const float c_lo = 1.0f - 0x1p-22f, c_hi = 1.0f + 0x1p-22f;
    long long total = 0, bad_mk = 0, bad_br = 0, fallback = 0, bad_plain = 0;
#pragma omp parallel for reduction(+ : total, bad_mk, bad_br, fallback, bad_plain) schedule(dynamic, 32)
    for (int mb = 1; mb < 0x7c00; ++mb) {
        const float m = h2f((uint16_t)mb);
        const float s = m / 127.0f;
        const float inv = 1.0f / s;
        const float inv_lo = inv * c_lo, inv_hi = inv * c_hi;
        for (int vb = 0; vb < 0x10000; ++vb) {
            if (((vb >> 10) & 0x1f) == 0x1f) continue; /* inf, NaN */
            if ((vb & 0x7fff) > mb) continue;           /* |v| > m */
            const float v = h2f((uint16_t)vb);
            const float q = rintf(v / s);
            const int ref = (int)fmaxf(-127.0f, fminf(127.0f, q));
            const float z = v * inv;
            const float r = fmaf(-z, s, v);
            const float z1 = fmaf(r, inv, z);
            if (low_code(z1 + M) != ref) ++bad_mk;
            if (low_code(z + M) != ref) ++bad_plain;
            const float tl = fmaf(v, inv_lo, M), th = fmaf(v, inv_hi, M);
            if (tl == th) {
                if (low_code(tl) != ref) ++bad_br;
            } else {
                ++fallback;
            }
            ++total;
        }
    }
    printf("pairs %lld markstein_wrong %lld plain_wrong %lld bracket_wrong %lld bracket_undecided %lld\n", total,
           bad_mk, bad_plain, bad_br, fallback);
    return (bad_mk || bad_br) ? 1 : 0;
}
