/* ng_oracle.c - CPU restatement of the reference's per-layer kernel semantics.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker for the gfx950 library:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it. The product path (neurogrid_amd) never calls it.
 *
 * Sources restated (reference paths relative to the reference checkout):
 *   gather      gpu/cuda/kernels.cu:669-685
 *   rmsnorm     gpu/cuda/kernels.cu:58-95, bf16_utils.cu:57-93,
 *               scripts/generate_golden.py:43-47
 *   add+norm    gpu/cuda/kernels.cu:196-235
 *   silu/mul    gpu/cuda/kernels.cu:126-188, 269-359; bf16_utils.cu:122-213;
 *               scripts/generate_golden.py:50-52
 *   rope        gpu/cuda/kernels.cu:371-489, bf16_utils.cu:330-378,
 *               scripts/generate_golden.py:55-77
 *   quantize    gpu/cuda/quantize.cu:59-95, 189-231, 274-316 (with
 *               round-half-to-even instead of roundf, and IEEE division)
 *   dequantize  gpu/cuda/quantize.cu:147-158, gpu/cuda/matmul.cu:169-187
 *   softmax     gpu/cuda/kernels.cu:580-631 (true row maximum)
 *
 * Arithmetic: IEEE fp32 with round-to-nearest-even, no contraction
 * (built with -ffp-contract=off), results rounded once to the 16-bit
 * element type. The RMSNorm statistic is RN_f32 of the exact sum of squares
 * (computed with 128-bit integers); see ora_sumsq.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

typedef unsigned __int128 u128;

enum { DT_F16 = 0, DT_BF16 = 1 };

/* ------------------------------------------------------------------------ */
/* 16-bit formats                                                             */
/* ------------------------------------------------------------------------ */

float ora_f16_to_f32(uint16_t h) {
    int e = (h >> 10) & 0x1f;
    int m = h & 0x3ff;
    float v;
    if (e == 0)
        v = ldexpf((float)m, -24);
    else if (e == 31)
        v = m ? NAN : INFINITY;
    else
        v = ldexpf((float)(m | 0x400), e - 25);
    return (h & 0x8000) ? -v : v;
}

/* Round an fp32 value to binary16, ties to even. Works on the value: find
 * the representable neighbours with frexp/ldexp and pick by exact comparison. */
uint16_t ora_f32_to_f16(float f) {
    uint16_t sign = signbit(f) ? 0x8000 : 0;
    float a = fabsf(f);
    if (isnan(f)) return (uint16_t)(sign | 0x7e00);
    if (a >= 65520.0f) return (uint16_t)(sign | 0x7c00);
    /* quantum of the binade: 2^-24 for subnormals, else 2^(exp-11) */
    int ex;
    frexpf(a, &ex); /* a = m 2^ex, m in [0.5, 1) */
    int qexp = ex - 11;
    if (qexp < -24) qexp = -24;
    float scaled = ldexpf(a, -qexp);          /* exact: a has <= 24 bits */
    float lo = floorf(scaled);
    float rem = scaled - lo;                  /* exact */
    float k = lo;
    if (rem > 0.5f || (rem == 0.5f && fmodf(lo, 2.0f) != 0.0f)) k = lo + 1.0f;
    /* k * 2^qexp is the rounded value; encode it */
    double v = ldexp((double)k, qexp);
    if (v >= 65520.0) return (uint16_t)(sign | 0x7c00);
    if (v < ldexp(1.0, -14)) return (uint16_t)(sign | (uint16_t)(v * ldexp(1.0, 24)));
    int e2;
    double mm = frexp(v, &e2); /* v = mm 2^e2, mm in [0.5,1) */
    int E = e2 - 1 + 15;
    int M = (int)(mm * 2048.0) - 1024;
    return (uint16_t)(sign | (E << 10) | M);
}

float ora_bf16_to_f32(uint16_t h) {
    uint32_t x = (uint32_t)h << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

uint16_t ora_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
    uint32_t lower = x & 0xffffu;
    uint32_t upper = x >> 16;
    if (lower > 0x8000u || (lower == 0x8000u && (upper & 1u))) upper += 1;
    return (uint16_t)upper;
}

static inline float ld(const uint16_t* p, size_t i, int dt) {
    return dt == DT_BF16 ? ora_bf16_to_f32(p[i]) : ora_f16_to_f32(p[i]);
}
static inline uint16_t rn(float v, int dt) { return dt == DT_BF16 ? ora_f32_to_bf16(v) : ora_f32_to_f16(v); }

void ora_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int ora_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* Sum of squares: RN_f32(exact sum v_i^2)                                    */
/* ------------------------------------------------------------------------ */

/* v^2 in units of 2^-48, when v = M 2^e exactly with e >= -24 and |v| < 2^20. */
static int sq_units(float v, u128* out) {
    *out = 0;
    if (v == 0.0f) return 1;
    if (!isfinite(v)) return 0;
    float a = fabsf(v);
    if (a >= 1048576.0f) return 0;
    int ex;
    float m = frexpf(a, &ex);                  /* a = m 2^ex, m in [0.5,1) */
    uint64_t M = (uint64_t)ldexpf(m, 24);      /* a = M 2^(ex-24), exact */
    int e = ex - 24;
    while ((M & 1u) == 0) {
        M >>= 1;
        ++e;
    }
    if (e < -24) return 0;
    *out = ((u128)(M * M)) << (2 * e + 48);
    return 1;
}

/* Round S * 2^-48 to fp32, ties to even. */
static float units_to_f32(u128 S) {
    if (S == 0) return 0.0f;
    int p = 127;
    while (((S >> p) & 1) == 0) --p;
    if (p < 24) return ldexpf((float)(uint32_t)S, -48);
    int sh = p - 23;
    u128 q = S >> sh;
    u128 r = S & (((u128)1 << sh) - 1);
    u128 half = (u128)1 << (sh - 1);
    if (r > half || (r == half && (q & 1))) q += 1;
    return ldexpf((float)(uint64_t)q, sh - 48); /* q <= 2^24: exact as float */
}

static int g_exact_only = 0;
void ora_set_exact_only(int on) { g_exact_only = on; }

/* ss over n values; when every value qualifies for the integer form the
 * result is RN_f32 of the exact sum. A fast fp64 pass decides most rows: if
 * the interval S (1 +- 2^(k-51)), k = ceil(log2 n), rounds to one fp32
 * value, that value is RN_f32(exact). */
float ora_sumsq(const float* v, int n) {
    double S = 0.0;
    for (int i = 0; i < n; ++i) S += (double)v[i] * (double)v[i];
    if (!isfinite(S)) return (float)S;
    if (!g_exact_only) {
        int k = 1;
        while ((1 << k) < n) ++k;
        double d = ldexp(S, k - 51);
        if ((float)(S - d) == (float)(S + d)) return (float)S;
    }
    u128 U = 0;
    for (int i = 0; i < n; ++i) {
        u128 t;
        if (!sq_units(v[i], &t)) return (float)S;
        U += t;
    }
    return units_to_f32(U);
}

/* ------------------------------------------------------------------------ */
/* RMSNorm family                                                             */
/* ------------------------------------------------------------------------ */

static float rms_factor(float ss, int H, float eps) { return 1.0f / sqrtf(ss / (float)H + eps); }

/* y = RN((x * r) * w) */
void ora_rmsnorm(uint16_t* y, const uint16_t* x, const uint16_t* w, int T, int H, float eps, int dt) {
#pragma omp parallel
    {
        float* s = (float*)malloc(sizeof(float) * (size_t)H);
#pragma omp for schedule(static)
        for (int t = 0; t < T; ++t) {
            const uint16_t* xr = x + (size_t)t * H;
            for (int i = 0; i < H; ++i) s[i] = ld(xr, i, dt);
            float r = rms_factor(ora_sumsq(s, H), H, eps);
            uint16_t* yr = y + (size_t)t * H;
            for (int i = 0; i < H; ++i) yr[i] = rn((s[i] * r) * ld(w, i, dt), dt);
        }
        free(s);
    }
}

/* s = x + res (fp32); res_out = RN(s); y = RN((res_out * r) * w), r from sum s^2.
 * Outputs may alias inputs row for row. */
void ora_add_rmsnorm(uint16_t* y, uint16_t* res_out, const uint16_t* x, const uint16_t* res, const uint16_t* w,
                     int T, int H, float eps, int dt) {
#pragma omp parallel
    {
        float* s = (float*)malloc(sizeof(float) * (size_t)H);
#pragma omp for schedule(static)
        for (int t = 0; t < T; ++t) {
            size_t off = (size_t)t * H;
            for (int i = 0; i < H; ++i) s[i] = ld(x + off, i, dt) + ld(res + off, i, dt);
            float r = rms_factor(ora_sumsq(s, H), H, eps);
            for (int i = 0; i < H; ++i) {
                uint16_t ro = rn(s[i], dt);
                res_out[off + i] = ro;
                y[off + i] = rn((ld(&ro, 0, dt) * r) * ld(w, i, dt), dt);
            }
        }
        free(s);
    }
}

/* ------------------------------------------------------------------------ */
/* int8 absmax quantisation                                                   */
/* ------------------------------------------------------------------------ */

static float scale_of(float m) {
    float s = m / 127.0f;
    return s == 0.0f ? 1.0f : s;
}

/* q = fmaxf(-127, fminf(127, rint(v / scale))), the reference's clamp order
 * (quantize.cu:92,228,313) with ties to even: C's fminf returns its other
 * operand for a NaN, so a NaN quotient (a NaN element, or inf / inf) gives
 * +127. The maxima below use fmaxf, which skips NaNs as the reference's
 * block_reduce_max does (quantize.cu:24-50). */
static int8_t code_of(float v, float scale) {
    float q = rintf(v / scale); /* default rounding mode: nearest, ties to even */
    q = fmaxf(-127.0f, fminf(127.0f, q));
    return (int8_t)q;
}

static void quant_row(int8_t* q, float* scale, const float* v, int n) {
    float m = 0.0f;
    for (int i = 0; i < n; ++i) m = fmaxf(m, fabsf(v[i]));
    float s = scale_of(m);
    *scale = s;
    for (int i = 0; i < n; ++i) q[i] = code_of(v[i], s);
}

void ora_quant_rows(int8_t* q, float* scales, const uint16_t* x, int rows, int cols) {
#pragma omp parallel
    {
        float* v = (float*)malloc(sizeof(float) * (size_t)cols);
#pragma omp for schedule(static)
        for (int r = 0; r < rows; ++r) {
            for (int i = 0; i < cols; ++i) v[i] = ora_f16_to_f32(x[(size_t)r * cols + i]);
            quant_row(q + (size_t)r * cols, scales + r, v, cols);
        }
        free(v);
    }
}

/* y = RMSNorm(x) rounded to fp16, then per-row quantisation of y. */
void ora_rmsnorm_quant(int8_t* q, float* scales, const uint16_t* x, const uint16_t* w, int T, int H, float eps) {
#pragma omp parallel
    {
        float* s = (float*)malloc(sizeof(float) * (size_t)H);
#pragma omp for schedule(static)
        for (int t = 0; t < T; ++t) {
            const uint16_t* xr = x + (size_t)t * H;
            for (int i = 0; i < H; ++i) s[i] = ora_f16_to_f32(xr[i]);
            float r = rms_factor(ora_sumsq(s, H), H, eps);
            for (int i = 0; i < H; ++i) s[i] = ora_f16_to_f32(ora_f32_to_f16((s[i] * r) * ora_f16_to_f32(w[i])));
            quant_row(q + (size_t)t * H, scales + t, s, H);
        }
        free(s);
    }
}

void ora_add_rmsnorm_quant(int8_t* q, float* scales, uint16_t* res_out, const uint16_t* x, const uint16_t* res,
                           const uint16_t* w, int T, int H, float eps) {
#pragma omp parallel
    {
        float* s = (float*)malloc(sizeof(float) * (size_t)H);
#pragma omp for schedule(static)
        for (int t = 0; t < T; ++t) {
            size_t off = (size_t)t * H;
            for (int i = 0; i < H; ++i) s[i] = ora_f16_to_f32(x[off + i]) + ora_f16_to_f32(res[off + i]);
            float r = rms_factor(ora_sumsq(s, H), H, eps);
            for (int i = 0; i < H; ++i) {
                uint16_t ro = ora_f32_to_f16(s[i]);
                res_out[off + i] = ro;
                s[i] = ora_f16_to_f32(ora_f32_to_f16((ora_f16_to_f32(ro) * r) * ora_f16_to_f32(w[i])));
            }
            quant_row(q + off, scales + t, s, H);
        }
        free(s);
    }
}

void ora_quant_tensor(int8_t* q, float* scale, const uint16_t* x, size_t n) {
    float m = 0.0f;
    for (size_t i = 0; i < n; ++i) m = fmaxf(m, fabsf(ora_f16_to_f32(x[i])));
    float s = scale_of(m);
    *scale = s;
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) q[i] = code_of(ora_f16_to_f32(x[i]), s);
}

void ora_quant_cols(int8_t* q, float* scales, const uint16_t* x, int K, int N) {
    for (int c = 0; c < N; ++c) scales[c] = 0.0f;
    for (int k = 0; k < K; ++k)
        for (int c = 0; c < N; ++c) scales[c] = fmaxf(scales[c], fabsf(ora_f16_to_f32(x[(size_t)k * N + c])));
    for (int c = 0; c < N; ++c) scales[c] = scale_of(scales[c]);
#pragma omp parallel for schedule(static)
    for (int k = 0; k < K; ++k)
        for (int c = 0; c < N; ++c) q[(size_t)k * N + c] = code_of(ora_f16_to_f32(x[(size_t)k * N + c]), scales[c]);
}

/* mode 0: scale per row, 1: per column, 2: one scale. out = RN_f16(RN_f32(q * s)). */
void ora_dequant(uint16_t* out, const int8_t* q, const float* scales, int rows, int cols, int mode) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) {
            float s = mode == 0 ? scales[r] : (mode == 1 ? scales[c] : scales[0]);
            size_t i = (size_t)r * cols + c;
            out[i] = ora_f32_to_f16((float)q[i] * s);
        }
}

/* ------------------------------------------------------------------------ */
/* Element-wise                                                               */
/* ------------------------------------------------------------------------ */

enum { OP_ADD = 0, OP_MUL = 1, OP_SILU = 2, OP_SILU_MUL = 3, OP_SCALE = 4 };

static float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

void ora_elementwise(uint16_t* out, const uint16_t* a, const uint16_t* b, float s, size_t n, int op, int dt) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) {
        float x = ld(a, i, dt);
        float v;
        switch (op) {
            case OP_ADD: v = x + ld(b, i, dt); break;
            case OP_MUL: v = x * ld(b, i, dt); break;
            case OP_SILU: v = x * sigmoidf_(x); break;
            case OP_SILU_MUL: v = (x * sigmoidf_(x)) * ld(b, i, dt); break;
            default: v = x * s; break;
        }
        out[i] = rn(v, dt);
    }
}

/* ------------------------------------------------------------------------ */
/* RoPE                                                                       */
/* ------------------------------------------------------------------------ */

void ora_rope_inv_freq(float* inv, int D, float theta) {
    for (int i = 0; i < D / 2; ++i) {
        float expo = (2.0f * (float)i) / (float)D;
        inv[i] = 1.0f / powf(theta, expo);
    }
}

/* in/out [T, nh, D]; style 1 pairs (2i, 2i+1), any other style (i, i + D/2). */
void ora_rope(uint16_t* out, const uint16_t* in, const int* pos, int T, int nh, int D, int style, float theta,
              int dt) {
    int half = D / 2;
    float* inv = (float*)malloc(sizeof(float) * (size_t)half);
    ora_rope_inv_freq(inv, D, theta);
#pragma omp parallel
    {
        float* cs = (float*)malloc(sizeof(float) * (size_t)D);
#pragma omp for schedule(static)
        for (int t = 0; t < T; ++t) {
            for (int i = 0; i < half; ++i) {
                float ang = (float)pos[t] * inv[i];
                cs[2 * i] = cosf(ang);
                cs[2 * i + 1] = sinf(ang);
            }
            for (int h = 0; h < nh; ++h) {
                size_t base = ((size_t)t * nh + h) * D;
                for (int i = 0; i < half; ++i) {
                    size_t i1 = style == 1 ? base + 2 * i : base + i;
                    size_t i2 = style == 1 ? base + 2 * i + 1 : base + i + half;
                    float c = cs[2 * i], s = cs[2 * i + 1];
                    float x1 = ld(in, i1, dt), x2 = ld(in, i2, dt);
                    float y1 = x1 * c - x2 * s;
                    float y2 = x1 * s + x2 * c;
                    out[i1] = rn(y1, dt);
                    out[i2] = rn(y2, dt);
                }
            }
        }
        free(cs);
    }
    free(inv);
}

/* ------------------------------------------------------------------------ */
/* Gather, softmax                                                            */
/* ------------------------------------------------------------------------ */

void ora_gather(uint16_t* out, const uint16_t* table, const int* ids, int T, int H) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t) memcpy(out + (size_t)t * H, table + (size_t)ids[t] * H, sizeof(uint16_t) * (size_t)H);
}

void ora_softmax(uint16_t* out, const uint16_t* in, int rows, int cols) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const uint16_t* x = in + (size_t)r * cols;
        float m = -INFINITY;
        for (int i = 0; i < cols; ++i) m = fmaxf(m, ora_f16_to_f32(x[i]));
        double s = 0.0;
        for (int i = 0; i < cols; ++i) s += exp((double)ora_f16_to_f32(x[i]) - m);
        for (int i = 0; i < cols; ++i)
            out[(size_t)r * cols + i] = ora_f32_to_f16((float)(exp((double)ora_f16_to_f32(x[i]) - m) / s));
    }
}

/* ------------------------------------------------------------------------ */
/* fp32-storage variants: the reference CPU golden path in fp32 (TinyLlama   */
/* configuration, scripts/generate_golden.py:43-77 in torch.float32).        */
/* ------------------------------------------------------------------------ */

void ora_rmsnorm_f32(float* y, const float* x, const float* w, int T, int H, float eps) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t) {
        const float* xr = x + (size_t)t * H;
        float r = rms_factor(ora_sumsq(xr, H), H, eps);
        for (int i = 0; i < H; ++i) y[(size_t)t * H + i] = (xr[i] * r) * w[i];
    }
}

void ora_elementwise_f32(float* out, const float* a, const float* b, float s, size_t n, int op) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) {
        float x = a[i];
        switch (op) {
            case OP_ADD: out[i] = x + b[i]; break;
            case OP_MUL: out[i] = x * b[i]; break;
            case OP_SILU: out[i] = x * sigmoidf_(x); break;
            case OP_SILU_MUL: out[i] = (x * sigmoidf_(x)) * b[i]; break;
            default: out[i] = x * s; break;
        }
    }
}

void ora_rope_f32(float* out, const float* in, const int* pos, int T, int nh, int D, int style, float theta) {
    int half = D / 2;
    float* inv = (float*)malloc(sizeof(float) * (size_t)half);
    ora_rope_inv_freq(inv, D, theta);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t) {
        for (int h = 0; h < nh; ++h) {
            size_t base = ((size_t)t * nh + h) * D;
            for (int i = 0; i < half; ++i) {
                float ang = (float)pos[t] * inv[i];
                float c = cosf(ang), s = sinf(ang);
                size_t i1 = style == 1 ? base + 2 * i : base + i;
                size_t i2 = style == 1 ? base + 2 * i + 1 : base + i + half;
                float x1 = in[i1], x2 = in[i2];
                out[i1] = x1 * c - x2 * s;
                out[i2] = x1 * s + x2 * c;
            }
        }
    }
    free(inv);
}

/* bf16 -> fp16 the way the model loader converts a bf16 checkpoint on the host
 * (pkg/model/loader.go:23-85): widen to fp32 by a 16-bit shift (:30-32), then
 * float32ToFloat16Bits (:46-85): Inf -> 0x7C00, NaN -> 0x7E00 (sign kept),
 * exponent >= 31 after rebias -> Inf, rebias <= 0 -> subnormal by shifting
 * the mantissa with its hidden bit right (1 - exp16) and then 13 (zero below
 * -10), otherwise the mantissa truncated to 10 bits. */
static uint16_t loader_f32_to_f16(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    uint32_t sign = (bits >> 31) & 1u;
    int exp = (int)((bits >> 23) & 0xffu) - 127;
    uint32_t mant = bits & 0x7fffffu;
    if (exp == 128) return (uint16_t)((sign << 15) | (mant == 0 ? 0x7c00u : 0x7e00u));
    int exp16 = exp + 15;
    if (exp16 <= 0) {
        if (exp16 < -10) return (uint16_t)(sign << 15);
        mant = (mant | 0x800000u) >> (unsigned)(1 - exp16);
        return (uint16_t)((sign << 15) | (mant >> 13));
    }
    if (exp16 >= 31) return (uint16_t)((sign << 15) | 0x7c00u);
    return (uint16_t)((sign << 15) | ((uint32_t)exp16 << 10) | (mant >> 13));
}

void ora_bf16_to_f16_trunc(uint16_t* out, const uint16_t* in, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        uint32_t b = (uint32_t)in[i] << 16;
        float f;
        memcpy(&f, &b, 4);
        out[i] = loader_f32_to_f16(f);
    }
}

/* Row gather of any element size (bit copy). */
void ora_gather_bytes(void* out, const void* table, const int* ids, int T, size_t row_bytes) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t)
        memcpy((char*)out + (size_t)t * row_bytes, (const char*)table + (size_t)ids[t] * row_bytes, row_bytes);
}
